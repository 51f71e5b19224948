"""ctypes binding of libkvrepair.so (the gfx950 HIP kernels behind include/kvrepair.h).

The library is loaded lazily and only after ``import torch``: it links the HIP
runtime by SONAME, so the dynamic linker binds it to the runtime instance
torch already mapped and the two share streams and device memory. There is no
fallback: a missing or stale library raises immediately.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libkvrepair.so"
ABI_VERSION = 1

ATTN_ROUNDED_PROBABILITIES = 1  # kvr_attention_schedule_ex flag (include/kvrepair.h)
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_vpp = ctypes.POINTER(ctypes.c_void_p)

_lock = threading.Lock()
_lib = None


class NativeError(RuntimeError):
    """A kvrepair C entry point returned a negative status."""


class LayerDesc(ctypes.Structure):
    """Mirror of kvr_layer_desc (include/kvrepair.h)."""

    _fields_ = [(name, ctypes.c_void_p) for name in (
        "input_norm", "post_norm", "q_norm", "k_norm", "w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")] + \
        [(name, ctypes.c_int64) for name in ("ld_q", "ld_k", "ld_v", "ld_o", "ld_gate", "ld_up", "ld_down")] + \
        [(name, ctypes.c_float) for name in ("eps_input", "eps_post", "eps_q", "eps_k")] + \
        [("next_norm", ctypes.c_void_p), ("eps_next", ctypes.c_float), ("input_normed", ctypes.c_int32)] + \
        [("cache_k", ctypes.c_void_p), ("cache_v", ctypes.c_void_p), ("cache_strides", ctypes.c_int64 * 6)]


class RefreshDesc(ctypes.Structure):
    """Mirror of kvr_refresh_desc (include/kvrepair.h)."""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "rows", "hidden", "q_heads", "kv_heads", "head_dim", "intermediate")] + [
        ("n_keys", ctypes.c_int64), ("scale", ctypes.c_float), ("dtype", ctypes.c_int32),
        ("positions", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("cs_strides", ctypes.c_int64 * 4), ("schedule", ctypes.c_void_p), ("schedule_len", ctypes.c_int64),
        ("host_schedule", ctypes.c_void_p), ("attn_workspace", ctypes.c_void_p),
        ("attn_workspace_bytes", ctypes.c_int64), ("gemm_workspace", ctypes.c_void_p),
        ("gemm_workspace_bytes", ctypes.c_int64), ("scratch", ctypes.c_void_p), ("scratch_bytes", ctypes.c_int64)]


def _declare(lib: ctypes.CDLL) -> None:
    lib.kvr_abi_version.argtypes = []
    lib.kvr_abi_version.restype = ctypes.c_int
    lib.kvr_token_alignment.argtypes = [_vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int64, _i64p]
    lib.kvr_token_alignment.restype = ctypes.c_int
    lib.kvr_upload_async.argtypes = [_vp, _vpp, _i64p, ctypes.c_int32, _vp]
    lib.kvr_upload_async.restype = ctypes.c_int
    lib.kvr_status_string.argtypes = [ctypes.c_int]
    lib.kvr_status_string.restype = ctypes.c_char_p
    lib.kvr_rope_delta_rotate.argtypes = [_vpp, _vpp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                          ctypes.c_int32, ctypes.c_int32, _i64p, _i64p, ctypes.c_int64, _vp,
                                          ctypes.c_float, ctypes.c_int32, _vp]
    lib.kvr_rope_delta_rotate.restype = ctypes.c_int
    lib.kvr_shift_cache_build.argtypes = [_vpp, _vpp, _vpp, _vpp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_int32, _i64p, _i64p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_float,
                                          ctypes.c_int32, _vp]
    lib.kvr_shift_cache_build.restype = ctypes.c_int
    lib.kvr_indexed_scatter_kv.argtypes = [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                           ctypes.c_int32, _i64p, ctypes.c_int32, _vp]
    lib.kvr_indexed_scatter_kv.restype = ctypes.c_int
    lib.kvr_rope_scatter_kv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, _i64p, _i64p, ctypes.c_int32,
                                        _vp]
    lib.kvr_rope_scatter_kv.restype = ctypes.c_int
    lib.kvr_rope_scatter_kv_norm.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64,
                                             ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, _i64p,
                                             _i64p, _vp, _vp, ctypes.c_float, ctypes.c_float, ctypes.c_int32, _vp]
    lib.kvr_rope_scatter_kv_norm.restype = ctypes.c_int
    lib.kvr_rms_norm.argtypes = [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, _i64p, ctypes.c_float,
                                 ctypes.c_int32, _vp]
    lib.kvr_rms_norm.restype = ctypes.c_int
    lib.kvr_silu_mul.argtypes = [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, _vp]
    lib.kvr_silu_mul.restype = ctypes.c_int
    lib.kvr_linear_splits.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    lib.kvr_linear_splits.restype = ctypes.c_int32
    lib.kvr_linear_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    lib.kvr_linear_workspace_bytes.restype = ctypes.c_int64
    lib.kvr_linear.argtypes = [_vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                               ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int32, _vp]
    lib.kvr_linear.restype = ctypes.c_int
    lib.kvr_linear_multi.argtypes = [_vp, ctypes.c_int32, _vpp, _i32p, _i64p, _vp, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, _vp, ctypes.c_int64, _vp,
                                     ctypes.c_int64, ctypes.c_int32, _vp]
    lib.kvr_linear_multi.restype = ctypes.c_int
    lib.kvr_linear_multi_partials.argtypes = [_vp, ctypes.c_int32, _vpp, _i32p, _i64p, _vp, ctypes.c_int32,
                                              ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int64,
                                              ctypes.c_int32, _vp, _i32p]
    lib.kvr_linear_multi_partials.restype = ctypes.c_int
    lib.kvr_copy_kv_interval.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                         ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, _i64p, ctypes.c_int32, _vp]
    lib.kvr_copy_kv_interval.restype = ctypes.c_int
    lib.kvr_refresh_inputs.argtypes = [_vp, ctypes.c_int32, ctypes.c_int64, _vp, ctypes.c_int64, _vp, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_int32, _vp, ctypes.c_int64, _vp, ctypes.c_int32,
                                       ctypes.c_float, _vp, _vp, ctypes.c_int32, _vp]
    lib.kvr_refresh_inputs.restype = ctypes.c_int
    lib.kvr_query_relevance.argtypes = [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, _vp, ctypes.c_int32,
                                        ctypes.c_int64, _vp, ctypes.c_int32, ctypes.c_float, _vp, ctypes.c_int32, _vp]
    lib.kvr_query_relevance.restype = ctypes.c_int
    _desc_p = ctypes.POINTER(LayerDesc)
    _refresh_p = ctypes.POINTER(RefreshDesc)
    lib.kvr_decoder_scratch_bytes.argtypes = [_refresh_p]
    lib.kvr_decoder_scratch_bytes.restype = ctypes.c_int64
    lib.kvr_decoder_gemm_workspace_bytes.argtypes = [_refresh_p]
    lib.kvr_decoder_gemm_workspace_bytes.restype = ctypes.c_int64
    lib.kvr_decoder_layer.argtypes = [_desc_p, _refresh_p, _vp, _vp]
    lib.kvr_decoder_layer.restype = ctypes.c_int
    lib.kvr_decoder_forward.argtypes = [_desc_p, ctypes.c_int32, _refresh_p, _vp, _vp]
    lib.kvr_decoder_forward.restype = ctypes.c_int
    lib.kvr_decoder_desc_sizes.argtypes = [_i64p]
    lib.kvr_decoder_desc_sizes.restype = None
    lib.kvr_attention_schedule.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _i32p, ctypes.c_int64]
    lib.kvr_attention_schedule.restype = ctypes.c_int64
    lib.kvr_attention_schedule_ex.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _i32p,
                                              ctypes.c_int64]
    lib.kvr_attention_schedule_ex.restype = ctypes.c_int64
    lib.kvr_attention_workspace_bytes.argtypes = [_i32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
    lib.kvr_attention_workspace_bytes.restype = ctypes.c_int64
    lib.kvr_packed_causal_attention.argtypes = [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32,
                                                ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
                                                _i64p, _vp, ctypes.c_int64, _i32p, _vp, ctypes.c_int64,
                                                ctypes.c_int32, _vp]
    lib.kvr_packed_causal_attention.restype = ctypes.c_int
    lib.kvr_packed_causal_attention_noalloc.argtypes = [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32,
                                                        ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                                        ctypes.c_float, _i64p, _vp, ctypes.c_int64, _i32p,
                                                        ctypes.c_int32, _vp]
    lib.kvr_packed_causal_attention_noalloc.restype = ctypes.c_int
    lib.kvr_attention_scratch_limit.argtypes = []
    lib.kvr_attention_scratch_limit.restype = ctypes.c_int64


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it is missing or has another ABI version."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if torch.version.hip is None:
                raise NativeError("libkvrepair requires a ROCm build of PyTorch")
            if not LIB_PATH.exists():
                raise NativeError(f"{LIB_PATH} is missing; build it with `python __graft_entry__.py` "
                                  "(budgeted-kv-cache-repair_amd/build_lib.py)")
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            version = handle.kvr_abi_version()
            if version != ABI_VERSION:
                raise NativeError(f"libkvrepair ABI {version} != expected {ABI_VERSION}; rebuild the library")
            sizes = (ctypes.c_int64 * 2)()
            handle.kvr_decoder_desc_sizes(sizes)
            if tuple(sizes) != (ctypes.sizeof(LayerDesc), ctypes.sizeof(RefreshDesc)):
                raise NativeError(f"libkvrepair descriptor sizes {tuple(sizes)} do not match the bindings; rebuild")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status < 0:
        text = lib().kvr_status_string(int(status)).decode()
        raise NativeError(f"{what} failed: {text} (status {status})")


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    """hipStream_t of the caller's current stream on ``device``."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def i64_array(values) -> ctypes.Array:
    values = list(values)
    return (ctypes.c_int64 * len(values))(*values)


def ptr_array(tensors) -> ctypes.Array:
    tensors = list(tensors)
    return (ctypes.c_void_p * len(tensors))(*(t.data_ptr() for t in tensors))


def strides3(t: torch.Tensor) -> list[int]:
    """{head, row, dim} element strides of a [1, heads, rows, dim] tensor."""
    return [int(t.stride(1)), int(t.stride(2)), int(t.stride(3))]
