"""Positional correction of a stale KV cache on MI355X.

Drop-in counterparts of the reference cache operators
(src/kv_cache_repair/cache.py): ``shifted_suffix_keys`` (RoPE delta rotation,
:47-77), ``build_halo_cache`` (:103-144) and ``clone_cache`` (:31-44). The
rotation and every full-cache copy run in libkvrepair: one launch covers all
layers, K and V together, where the reference issues ~10 eager kernels plus
two concatenations per layer. Caches are transformers 5.15 ``DynamicCache``
objects whose layers hold ``[1, kv_heads, tokens, head_dim]`` tensors.
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from . import _native
from .alignment import token_alignment, token_alignment_host
from .kernels.executor import layer_kv, tensor_layout


class OperatorShim:
    """The small model surface the repair operators use (reference cache.py:13-22)."""

    def __init__(self, model: Any, tokenizer: Any = None) -> None:
        self.generator = model
        self.tokenizer = tokenizer

    @staticmethod
    def _base_transformer(model: Any) -> Any:
        return getattr(model, "base_model", model)


def cache_from_tensors(pairs) -> DynamicCache:
    """A DynamicCache whose layers hold exactly these tensors (no copy, no cat)."""
    cache = DynamicCache()
    for key, value in pairs:
        layer = DynamicLayer()
        layer.keys, layer.values = key, value
        layer.dtype, layer.device = key.dtype, key.device
        layer.is_initialized = True
        cache.layers.append(layer)
    return cache


def _require_device(tensor: torch.Tensor, what: str) -> None:
    if not tensor.is_cuda or torch.version.hip is None:
        raise ValueError(f"{what} runs on a ROCm GPU device; got a {tensor.device.type} tensor")
    if tensor.dtype not in _native.DTYPE_CODES:
        raise ValueError(f"{what} supports float32, float16 and bfloat16 caches")


def _rotary(model: Any, device: torch.device):
    """(inv_freq fp32 on device, attention_scaling, rotary_dim) of the model's RoPE."""
    rotary = OperatorShim._base_transformer(model).rotary_emb
    inv_freq = rotary.inv_freq.to(device=device, dtype=torch.float32)
    return inv_freq.contiguous(), float(getattr(rotary, "attention_scaling", 1.0)), 2 * int(inv_freq.numel())


def _vocab_size(model: Any) -> int | None:
    """Rows of the model's input embedding table, or None when it has none."""
    get = getattr(model, "get_input_embeddings", None)
    weight = getattr(get(), "weight", None) if callable(get) else None
    return int(weight.shape[0]) if isinstance(weight, torch.Tensor) and weight.ndim == 2 else None


def _shift_launcher(old_k, old_v, new_k, new_v, *, inv_freq, scaling, rotary_dim):
    """kvr_shift_cache_build over lists of per-layer tensors, with every pointer
    and stride argument bound now; the returned function takes the row ranges
    and the shift and launches (one launch per 64 layers)."""
    first = old_k[0]
    _, heads, _, dim = first.shape
    fixed = (_native.ptr_array(old_k), _native.ptr_array(old_v), _native.ptr_array(new_k), _native.ptr_array(new_v),
             len(old_k), int(heads), int(dim), int(rotary_dim), _native.i64_array(_native.strides3(first)),
             _native.i64_array(_native.strides3(new_k[0])))
    tail = (inv_freq.data_ptr() if inv_freq is not None else None, float(scaling), _native.DTYPE_CODES[first.dtype],
            _native.stream_handle(first.device))
    build = _native.lib().kvr_shift_cache_build

    def launch(*, prefix_rows, old_tail_start, new_tail_start, tail_rows, shift) -> None:
        status = build(*fixed, int(prefix_rows), int(old_tail_start), int(new_tail_start), int(tail_rows),
                       int(shift), *tail)
        _native.check(status, "kvr_shift_cache_build")
    return launch


def _shift_rows(old_k, old_v, new_k, new_v, *, prefix_rows, old_tail_start, new_tail_start, tail_rows, shift,
                inv_freq, scaling, rotary_dim) -> None:
    """kvr_shift_cache_build over lists of per-layer tensors (one launch per 64 layers)."""
    _shift_launcher(old_k, old_v, new_k, new_v, inv_freq=inv_freq, scaling=scaling, rotary_dim=rotary_dim)(
        prefix_rows=prefix_rows, old_tail_start=old_tail_start, new_tail_start=new_tail_start, tail_rows=tail_rows,
        shift=shift)


def _check_uniform(pairs, what: str):
    first = pairs[0][0]
    # Fast path: every tensor has the first one's exact shape, strides, dtype and
    # GPU (what build_halo_cache and the executors produce) and that layout
    # passes the checks below; anything else takes the per-tensor checks.
    sig = (first.shape, first.stride(), first.dtype, first.get_device())
    if (first.ndim == 4 and first.shape[0] == 1 and sig[3] >= 0 and all(s > 0 for s in sig[1])
            and all((t.shape, t.stride(), t.dtype, t.get_device()) == sig for pair in pairs for t in pair)):
        _require_device(first, what)
        return
    for key, value in pairs:
        for t in (key, value):
            if t.ndim != 4 or t.shape[0] != 1 or t.shape[1] != first.shape[1] or t.shape[3] != first.shape[3]:
                raise ValueError(f"{what}: every layer must be [1, kv_heads, tokens, head_dim] with one geometry")
            if t.dtype != first.dtype or t.device != first.device:
                raise ValueError(f"{what}: every layer must share dtype and device")
            if t.stride() != first.stride() or any(s <= 0 for s in t.stride()):
                raise ValueError(f"{what}: every layer must share one positive stride layout")
        if key.shape != value.shape:
            raise ValueError(f"{what}: K and V shapes differ")
    _require_device(first, what)


@torch.no_grad()
def clone_cache(cache: Any, length: int | None = None) -> DynamicCache:
    """Clone all layers, optionally keeping only a prefix; never alias storage.

    One libkvrepair launch copies K and V of every layer (bit copy).
    """
    layers = [layer_kv(cache, i) for i in range(len(cache.layers))]
    if length is not None and (int(length) < 0 or (layers and int(length) > layers[0][0].shape[2])):
        raise ValueError("prefix length is outside the cache")
    if not layers:
        return DynamicCache()
    _check_uniform(layers, "clone_cache")
    rows = layers[0][0].shape[2] if length is None else int(length)
    shape = (1, layers[0][0].shape[1], rows, layers[0][0].shape[3])
    new = [(torch.empty(shape, dtype=k.dtype, device=k.device), torch.empty(shape, dtype=k.dtype, device=k.device))
           for k, _ in layers]
    if rows:
        _shift_rows([k for k, _ in layers], [v for _, v in layers], [k for k, _ in new], [v for _, v in new],
                    prefix_rows=rows, old_tail_start=0, new_tail_start=rows, tail_rows=0, shift=0, inv_freq=None,
                    scaling=1.0, rotary_dim=shape[3])
    return cache_from_tensors(new)


@torch.no_grad()
def shifted_suffix_keys(model: Any, key: torch.Tensor, shift: int) -> torch.Tensor:
    """RoPE delta re-rotation of one layer's retained-suffix keys (reference cache.py:47-77).

    ``model`` is an OperatorShim (or anything with ``generator``). Returns a new
    contiguous ``[1, kv_heads, rows, head_dim]`` tensor equal to the eager
    ``key * cos + rotate_half(key) * sin`` with cos/sin of ``inv_freq * shift``
    cast to the key dtype; ``shift == 0`` returns a bit-exact clone.
    """
    if key.ndim != 4 or key.shape[0] != 1:
        raise ValueError("key must be [1, kv_heads, rows, head_dim]")
    _require_device(key, "shifted_suffix_keys")
    out = torch.empty(key.shape, dtype=key.dtype, device=key.device)
    if not key.shape[2]:
        return out
    generator = getattr(model, "generator", model)
    inv_freq, scaling, rotary_dim = _rotary(generator, key.device)
    lib = _native.lib()
    status = lib.kvr_rope_delta_rotate(
        _native.ptr_array([key]), _native.ptr_array([out]), 1, int(key.shape[1]), int(key.shape[2]),
        int(key.shape[3]), int(rotary_dim), _native.i64_array(_native.strides3(key)),
        _native.i64_array(_native.strides3(out)), int(shift), inv_freq.data_ptr(), scaling,
        _native.DTYPE_CODES[key.dtype], _native.stream_handle(key.device))
    _native.check(status, "kvr_rope_delta_rotate")
    return out


def rope_delta_rotate_(keys: list[torch.Tensor], outs: list[torch.Tensor], shift: int, inv_freq: torch.Tensor,
                       attention_scaling: float = 1.0, rotary_dim: int | None = None) -> None:
    """Rotate the suffix keys of many layers in one launch: ``outs[l] = R(shift) keys[l]``.

    ``keys``/``outs`` are per-layer ``[1, kv_heads, rows, head_dim]`` views with
    one shared stride layout each; ``inv_freq`` is the fp32 device vector of
    the model's rotary frequencies. Writes only ``outs``.
    """
    if len(keys) != len(outs) or not keys:
        raise ValueError("keys and outs must be equal-length nonempty lists")
    _check_uniform(list(zip(keys, keys)), "rope_delta_rotate_")
    _check_uniform(list(zip(outs, outs)), "rope_delta_rotate_")
    if outs[0].shape != keys[0].shape:
        raise ValueError("rope_delta_rotate_: outs must match keys in shape")
    if inv_freq.dtype != torch.float32 or inv_freq.device != keys[0].device or not inv_freq.is_contiguous():
        raise ValueError("inv_freq must be a contiguous float32 tensor on the keys' device")
    rd = 2 * int(inv_freq.numel()) if rotary_dim is None else int(rotary_dim)
    first = keys[0]
    status = _native.lib().kvr_rope_delta_rotate(
        _native.ptr_array(keys), _native.ptr_array(outs), len(keys), int(first.shape[1]), int(first.shape[2]),
        int(first.shape[3]), rd, _native.i64_array(_native.strides3(first)),
        _native.i64_array(_native.strides3(outs[0])), int(shift), inv_freq.data_ptr(), float(attention_scaling),
        _native.DTYPE_CODES[first.dtype], _native.stream_handle(first.device))
    _native.check(status, "kvr_rope_delta_rotate")


@torch.no_grad()
def run_tokens_from_prefix(model: Any, prefix_cache: Any, input_ids: torch.Tensor, end_position: int) -> Any:
    """Native HF forward of boundary tokens after a prefix cache (reference cache.py:80-100)."""
    if not int(input_ids.shape[1]):
        return prefix_cache
    mask = torch.ones((1, int(end_position)), dtype=torch.long, device=input_ids.device)
    base = OperatorShim._base_transformer(getattr(model, "generator", model))
    return base(input_ids=input_ids, attention_mask=mask, past_key_values=prefix_cache, use_cache=True,
                return_dict=True).past_key_values


def _layer_addresses(cache: Any, what: str):
    """(first K tensor, K address array, V address array) of every cache layer,
    after _check_uniform's checks. The layout and addresses of all layers are
    read in one _kvr_layout pass; a cache that is not one uniform GPU layout
    takes _check_uniform's per-tensor path (same errors)."""
    k_bytes, v_bytes, first, uniform = tensor_layout().kv_layers(cache.layers)
    if not (uniform and first.ndim == 4 and first.shape[0] == 1 and first.get_device() >= 0
            and all(s > 0 for s in first.stride())):
        pairs = [layer_kv(cache, i) for i in range(len(cache.layers))]
        _check_uniform(pairs, what)
        return pairs[0][0], _native.ptr_array(k for k, _ in pairs), _native.ptr_array(v for _, v in pairs)
    _require_device(first, what)
    count = len(k_bytes) // 8
    return (first, (ctypes.c_void_p * count).from_buffer_copy(k_bytes),
            (ctypes.c_void_p * count).from_buffer_copy(v_bytes))


def _host_id_rows(old_input_ids: torch.Tensor, new_input_ids: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """Both id rows as int64 host arrays: CPU tensors are read in place (no copy,
    no device synchronisation, as the API layer holds its tokenizer ids); device
    ids come over in one device-to-host copy of both rows."""
    if old_input_ids.device.type == "cpu" and new_input_ids.device.type == "cpu":
        return (np.asarray(old_input_ids.numpy()[0], dtype=np.int64).reshape(-1),
                np.asarray(new_input_ids.numpy()[0], dtype=np.int64).reshape(-1))
    old_row, new_row = old_input_ids[0].reshape(-1), new_input_ids[0].reshape(-1)
    ids = torch.cat((old_row, new_row.to(device=old_row.device, dtype=old_row.dtype))).cpu().numpy()
    return ids[:old_row.numel()].astype(np.int64, copy=False), ids[old_row.numel():].astype(np.int64, copy=False)


@torch.no_grad()
def build_halo_cache(model: Any, old_cache: Any, old_input_ids: torch.Tensor, new_input_ids: torch.Tensor,
                     halo_tokens: int) -> tuple[DynamicCache, dict[str, int]]:
    """Keep the common prefix, recompute changed tokens and halo, shift the tail.

    Same result and metadata as the reference (cache.py:103-144). When no token
    needs recomputation the whole shifted cache (prefix copy, rotated K tail,
    copied V tail, every layer) is written by ONE kvr_shift_cache_build launch
    into one freshly allocated slab of independently owned per-layer tensors;
    the old cache is never mutated. The alignment (and the check that every id
    indexes the model's embedding table) is one host call on the id rows; the
    launch takes the per-layer output addresses computed from the slab, and the
    per-layer tensor views are made after it, while the GPU runs.
    """
    n_new = int(new_input_ids.shape[1])
    k0, old_k, old_v = _layer_addresses(old_cache, "build_halo_cache")
    generator = getattr(model, "generator", model)
    old_np, new_np = _host_id_rows(old_input_ids, new_input_ids)
    # the refresh and any boundary recomputation gather embedding rows by these
    # ids on the GPU: out-of-range ids are refused here, before any launch
    align = token_alignment_host(old_np, new_np, _vocab_size(generator))
    halo = min(max(int(halo_tokens), 0), align["suffix"])
    recompute_end = align["new_suffix_start"] + halo
    old_tail_start = align["old_suffix_start"] + halo
    tail_rows = align["suffix"] - halo
    inv_freq, scaling, rotary_dim = _rotary(generator, k0.device)
    layers, heads, dim = len(old_k), int(k0.shape[1]), int(k0.shape[3])
    # one allocation for every layer's K and V; layer l's K is block 2 l, its V block 2 l + 1
    slab = torch.empty((layers, 2, 1, heads, n_new, dim), dtype=k0.dtype, device=k0.device)
    if recompute_end == align["prefix"]:
        # No recomputed rows: prefix copy + shifted tail in one launch.
        if n_new:
            block = heads * n_new * dim * slab.element_size()
            base = slab.data_ptr()
            new_k = (ctypes.c_void_p * layers)(*range(base, base + 2 * layers * block, 2 * block))
            new_v = (ctypes.c_void_p * layers)(*range(base + block, base + 2 * layers * block, 2 * block))
            status = _native.lib().kvr_shift_cache_build(
                old_k, old_v, new_k, new_v, layers,
                heads, dim, int(rotary_dim), _native.i64_array(_native.strides3(k0)),
                _native.i64_array((n_new * dim, dim, 1)), align["prefix"], old_tail_start, recompute_end, tail_rows,
                align["position_shift"], inv_freq.data_ptr(), float(scaling), _native.DTYPE_CODES[k0.dtype],
                _native.stream_handle(k0.device))
            _native.check(status, "kvr_shift_cache_build")
        views = slab.view(2 * layers, 1, heads, n_new, dim).unbind(0)
    else:
        views = slab.view(2 * layers, 1, heads, n_new, dim).unbind(0)
        new_k, new_v = list(views[0::2]), list(views[1::2])
        prefix_cache = clone_cache(old_cache, align["prefix"])
        recomputed = run_tokens_from_prefix(generator, prefix_cache,
                                            new_input_ids[:, align["prefix"]:recompute_end].to(k0.device),
                                            recompute_end)
        old = [layer_kv(old_cache, i) for i in range(layers)]
        rec = [layer_kv(recomputed, i) for i in range(layers)]
        _check_uniform(rec, "build_halo_cache")
        _shift_rows([k for k, _ in rec], [v for _, v in rec], new_k, new_v,
                    prefix_rows=recompute_end, old_tail_start=0, new_tail_start=recompute_end, tail_rows=0, shift=0,
                    inv_freq=None, scaling=1.0, rotary_dim=rotary_dim)
        if tail_rows:
            _shift_rows([k for k, _ in old], [v for _, v in old], new_k, new_v, prefix_rows=0,
                        old_tail_start=old_tail_start, new_tail_start=recompute_end, tail_rows=tail_rows,
                        shift=align["position_shift"], inv_freq=inv_freq, scaling=scaling, rotary_dim=rotary_dim)
    return cache_from_tensors(zip(views[0::2], views[1::2])), {
        **align, "halo_tokens": halo, "recomputed_tokens": align["mandatory_changed_tokens"] + halo}


def merge_intervals(intervals: list[tuple[int, int]]) -> list[tuple[int, int]]:
    """Union of half-open intervals as sorted maximal runs (reference cache.py:195-204)."""
    merged: list[tuple[int, int]] = []
    for start, end in sorted((int(s), int(e)) for s, e in intervals if int(e) > int(s)):
        if merged and start <= merged[-1][1]:
            merged[-1] = (merged[-1][0], max(merged[-1][1], end))
        else:
            merged.append((start, end))
    return merged
