"""Validated plans and gfx950 operators for selected-query causal attention.

Public names, argument meaning and error classes follow the reference operator
module (src/kv_cache_repair/kernels/indexed_attention.py): ``IndexedPlan``,
``DeviceIndexedPlan``, ``indexed_kv_scatter_`` and ``indexed_causal_attention``.
The device code is libkvrepair (HIP, gfx950) instead of Triton.

The host plan owns immutable integer metadata and is uploaded once per request.
Device-plan tensors are read-only by contract. No API copies metadata back to
the host. Scatter and attention run on the caller's current stream, so they are
ordered with each other and with surrounding torch work on that stream.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from functools import lru_cache
from numbers import Integral, Real
from typing import Sequence

import torch

from .. import _native
from .writeback import _nonoverlapping_layout

BLOCK_M = 16
BLOCK_N = 64
_DTYPES = (torch.float16, torch.bfloat16)
_NATIVE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_TARGET_ARCH = "gfx950"


@lru_cache(maxsize=32)
def _device_arch(device_index: int) -> str:
    """Cache host device properties only; never a request or tensor."""
    return str(torch.cuda.get_device_properties(device_index).gcnArchName)


def _require_gfx950(device: torch.device) -> None:
    """The library carries gfx950 code objects only; refuse anything else up front."""
    if torch.version.hip is None or device.type != "cuda" or device.index is None:
        raise ValueError("indexed HIP kernels require an AMD ROCm (CUDA-API) device")
    if not _device_arch(device.index).startswith(_TARGET_ARCH):
        raise ValueError(f"indexed HIP kernels require an AMD {_TARGET_ARCH} (MI355X) device")


@dataclass(frozen=True)
class IndexedPlan:
    """Sorted absolute positions, validated entirely on the CPU.

    Tensor positions are rejected: building a plan must not hide a
    device-to-host synchronisation (reference indexed_attention.py:42-83).
    ``full_prefix_tiles``/``total_tiles`` are the per-16-row key-block bounds
    of the reference plan: (first + 1) // 64 and (last + 64) // 64.
    """

    positions: Sequence[int]
    logical_length: int
    full_prefix_tiles: tuple[int, ...] = field(init=False)
    total_tiles: tuple[int, ...] = field(init=False)

    def __post_init__(self):
        if isinstance(self.logical_length, bool) or not isinstance(self.logical_length, Integral):
            raise ValueError("logical_length must be a host integer")
        length = int(self.logical_length)
        if length < 0 or length > (1 << 63) - 1:
            raise ValueError("logical_length must fit nonnegative signed int64")
        if isinstance(self.positions, torch.Tensor):
            raise ValueError("positions must be host integers, not a tensor")
        try:
            raw = tuple(self.positions)
        except TypeError as error:
            raise ValueError("positions must be a sequence of host integers") from error
        if all(type(p) is int for p in raw):  # plain ints (the common case): no ABC checks
            positions = raw
        else:
            if any(isinstance(p, bool) or not isinstance(p, Integral) for p in raw):
                raise ValueError("positions must contain host integers")
            positions = tuple(int(p) for p in raw)
        if positions and (min(positions) < 0 or max(positions) >= length):
            raise ValueError("positions must lie within logical_length")
        if any(b <= a for a, b in zip(positions, positions[1:])):
            raise ValueError("positions must be strictly increasing and unique")
        full = tuple((positions[i] + 1) // BLOCK_N for i in range(0, len(positions), BLOCK_M))
        total = tuple((positions[min(i + BLOCK_M, len(positions)) - 1] + BLOCK_N) // BLOCK_N
                      for i in range(0, len(positions), BLOCK_M))
        object.__setattr__(self, "positions", positions)
        object.__setattr__(self, "logical_length", length)
        object.__setattr__(self, "full_prefix_tiles", full)
        object.__setattr__(self, "total_tiles", total)

    @property
    def selected_count(self) -> int:
        return len(self.positions)

    def to(self, device: torch.device | str | int, *, attention: tuple | None = None) -> "DeviceIndexedPlan":
        """Upload O(B) metadata on the caller's current stream for this device.

        ``attention`` = (n_q_heads, n_kv_heads, head_dim, dtype, rounded) also
        builds that attention work schedule (DeviceIndexedPlan.attention_schedule)
        and uploads it in the same copy."""
        device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
        if device.type != "cuda":
            raise ValueError("device plan requires a CUDA (ROCm) device")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        # int64 positions and bounds; version counters stay live even under
        # inference mode so every launch can reject in-place mutation with a
        # host-side check instead of a device read.
        # One upload for the three arrays (and the schedule) through the
        # library's pinned staging (kvr_upload_async); the device tensors are
        # contiguous views of it (sharing one version counter, so a write
        # through any of them unseals the plan).
        n, tiles = len(self.positions), len(self.full_prefix_tiles)
        values = (ctypes.c_int64 * (n + 2 * tiles))(*self.positions, *self.full_prefix_tiles, *self.total_tiles)
        parts = [values]
        schedule = None
        if attention is not None:
            n_q_heads, n_kv_heads, head_dim, dtype, rounded = attention
            key = _schedule_key(n_q_heads, n_kv_heads, head_dim, dtype, 0, rounded)
            schedule = (key, _host_schedule(self, key, values))
            parts.append(schedule[1])
        with torch.inference_mode(False):
            both = _upload(parts, device)
            head = ctypes.sizeof(values)
            packed = both[:head].view(torch.int64)
            positions, full, total = packed[:n], packed[n:n + tiles], packed[n + tiles:]
            sched_dev = both[head:].view(torch.int32) if schedule is not None else None
        tensors = (positions, full, total)
        seal = (id(self), tuple(id(t) for t in tensors), tuple(t._version for t in tensors))
        plan = DeviceIndexedPlan(self, positions, full, total, seal)
        if schedule is not None:
            plan._schedules[schedule[0]] = (schedule[1], sched_dev, sched_dev._version)
        return plan


def _schedule_key(n_q_heads, n_kv_heads, head_dim, dtype, chunk_keys, rounded) -> tuple:
    return (int(n_q_heads), int(n_kv_heads), int(head_dim), dtype, int(chunk_keys), bool(rounded))


def _host_schedule(host_plan: "IndexedPlan", key: tuple, positions=None):
    """kvr_attention_schedule_ex of ``host_plan`` for ``key`` (a _schedule_key): the
    int32 host array. ``positions``: the plan's positions as a ctypes int64
    array (its first selected_count entries), when the caller has one."""
    n_q_heads, n_kv_heads, head_dim, dtype, chunk_keys, rounded = key
    lib = _native.lib()
    pos = _native.i64_array(host_plan.positions) if positions is None else positions
    args = (pos, host_plan.selected_count, host_plan.logical_length, n_q_heads, n_kv_heads, head_dim,
            _native.DTYPE_CODES[dtype], chunk_keys, _native.ATTN_ROUNDED_PROBABILITIES if rounded else 0)
    need = lib.kvr_attention_schedule_ex(*args, None, 0)
    _native.check(int(need), "kvr_attention_schedule_ex")
    host = (ctypes.c_int32 * int(need))()
    _native.check(int(lib.kvr_attention_schedule_ex(*args, host, int(need))), "kvr_attention_schedule_ex")
    return host


def _upload(parts, device: torch.device) -> torch.Tensor:
    """A uint8 tensor on ``device`` holding the host buffers ``parts`` (ctypes
    arrays) back to back: one kvr_upload_async copy on the device's current
    stream from the library's pinned staging, so the host does not wait and the
    refresh's kernels can be enqueued while earlier work is still running."""
    sizes = [ctypes.sizeof(part) for part in parts]
    out = torch.empty(sum(sizes), dtype=torch.uint8, device=device)
    count = len(parts)
    status = _native.lib().kvr_upload_async(out.data_ptr(), (ctypes.c_void_p * count)(*map(ctypes.addressof, parts)),
                                            (ctypes.c_int64 * count)(*sizes), count, _native.stream_handle(device))
    _native.check(status, "kvr_upload_async")
    return out


@dataclass(frozen=True)
class DeviceIndexedPlan:
    """Device metadata from IndexedPlan.to; tensors are immutable by contract.

    Besides the reference's three arrays it caches, per (query heads, KV heads,
    head_dim, dtype), the attention work schedule: an int32 array computed on
    the host by kvr_attention_schedule and uploaded once.
    """

    host_plan: IndexedPlan
    positions: torch.Tensor
    full_prefix_tiles: torch.Tensor
    total_tiles: torch.Tensor
    _seal: tuple | None = field(default=None, repr=False, compare=False)
    _schedules: dict = field(default_factory=dict, repr=False, compare=False)

    @property
    def logical_length(self) -> int:
        return self.host_plan.logical_length

    @property
    def selected_count(self) -> int:
        return self.host_plan.selected_count

    @property
    def device(self) -> torch.device:
        return self.positions.device

    def attention_schedule(self, n_q_heads: int, n_kv_heads: int, head_dim: int, dtype: torch.dtype,
                           chunk_keys: int = 0, rounded: bool = False):
        """(host int32 array, device int32 tensor) work schedule for these shapes.

        rounded=True permits the kernel to round each softmax probability to
        the input dtype before the PV product (the SDPA precision the packed
        executor replaces); the default keeps them as a hi + lo pair.
        """
        key = _schedule_key(n_q_heads, n_kv_heads, head_dim, dtype, chunk_keys, rounded)
        cached = self._schedules.get(key)
        if cached is not None:
            host, dev, version = cached
            if dev._version != version:
                raise ValueError("device plan attention schedule was mutated")
            return host, dev
        host = _host_schedule(self.host_plan, key)
        with torch.inference_mode(False):
            dev = _upload([host], self.device).view(torch.int32)
        self._schedules[key] = (host, dev, dev._version)
        return host, dev


def _validate_plan(plan, device) -> None:
    if not isinstance(plan, DeviceIndexedPlan) or not isinstance(plan.host_plan, IndexedPlan):
        raise ValueError("device_plan must be produced by IndexedPlan.to")
    tiles = (plan.selected_count + BLOCK_M - 1) // BLOCK_M
    for tensor, count in ((plan.positions, plan.selected_count), (plan.full_prefix_tiles, tiles),
                          (plan.total_tiles, tiles)):
        if (not isinstance(tensor, torch.Tensor) or tensor.device != device or not tensor.is_cuda
                or tensor.dtype != torch.int64 or tensor.shape != (count,) or not tensor.is_contiguous()):
            raise ValueError("device plan has incompatible metadata shape, dtype, or device")
    tensors = (plan.positions, plan.full_prefix_tiles, plan.total_tiles)
    try:
        seal = (id(plan.host_plan), tuple(id(t) for t in tensors), tuple(t._version for t in tensors))
    except RuntimeError as error:
        raise ValueError("device plan must be produced by IndexedPlan.to") from error
    if plan._seal != seal:
        raise ValueError("device plan metadata was replaced, mutated, or not factory-created")


def _validate_tensors(tensors, dtypes=_DTYPES, dims=(64, 128)) -> None:
    if any(not isinstance(t, torch.Tensor) or t.ndim != 4 for t in tensors):
        raise ValueError("attention/cache tensors must have four dimensions")
    first = tensors[0]
    if not first.is_cuda or any(t.device != first.device for t in tensors):
        raise ValueError("all tensors must share one CUDA (ROCm) device")
    if first.dtype not in dtypes or any(t.dtype != first.dtype for t in tensors):
        names = ", ".join(str(d).replace("torch.", "") for d in dtypes)
        raise ValueError(f"all tensors must share one dtype among {names}")
    if any(t.shape[0] != 1 for t in tensors):
        raise ValueError("indexed kernels currently require batch size one")
    if any(t.shape[1] <= 0 or (dims is not None and t.shape[3] not in dims) for t in tensors):
        raise ValueError("head counts must be positive and head dimension must be 64 or 128")
    if any(any(s <= 0 for s in t.stride()) or not _nonoverlapping_layout(t) for t in tensors):
        raise ValueError("tensor layouts must have positive provably nonoverlapping strides")
    if any(t.requires_grad for t in tensors):
        raise ValueError("indexed kernels are inference-only; detach gradient-bearing inputs")


def _scatter_native(out_k, out_v, fresh_k, fresh_v, positions: torch.Tensor, n_sel: int) -> None:
    """Launch kvr_indexed_scatter_kv on the current stream (shapes already checked)."""
    _, heads, n_keys, dim = out_k.shape
    strides = _native.i64_array(_native.strides3(out_k) + _native.strides3(out_v) + _native.strides3(fresh_k)
                                + _native.strides3(fresh_v))
    status = _native.lib().kvr_indexed_scatter_kv(
        out_k.data_ptr(), out_v.data_ptr(), fresh_k.data_ptr(), fresh_v.data_ptr(), positions.data_ptr(),
        int(n_sel), int(heads), int(n_keys), int(dim), strides, _native.DTYPE_CODES[out_k.dtype],
        _native.stream_handle(out_k.device))
    _native.check(status, "kvr_indexed_scatter_kv")


def _rope_scatter_native(query, query_out, out_k, out_v, fresh_k, fresh_v, cos, sin, positions: torch.Tensor,
                        n_sel: int) -> None:
    """Launch kvr_rope_scatter_kv on the current stream (shapes already checked)."""
    _, hq, _, dim = query.shape
    _, hkv, n_keys, _ = out_k.shape
    strides = _native.i64_array(_native.strides3(query) + _native.strides3(query_out) + _native.strides3(fresh_k)
                                + _native.strides3(fresh_v) + _native.strides3(out_k) + _native.strides3(out_v))
    cs = _native.i64_array([int(cos.stride(-2)), int(cos.stride(-1)), int(sin.stride(-2)), int(sin.stride(-1))])
    status = _native.lib().kvr_rope_scatter_kv(
        query.data_ptr(), query_out.data_ptr(), fresh_k.data_ptr(), fresh_v.data_ptr(), out_k.data_ptr(),
        out_v.data_ptr(), cos.data_ptr(), sin.data_ptr(), positions.data_ptr(), int(n_sel), int(hq), int(hkv),
        int(n_keys), int(dim), strides, cs, _native.DTYPE_CODES[query.dtype], _native.stream_handle(query.device))
    _native.check(status, "kvr_rope_scatter_kv")


def _attention_native(q, k, v, out, device_plan: "DeviceIndexedPlan", scale: float) -> None:
    """Launch kvr_packed_causal_attention into ``out`` (shapes already checked)."""
    _, hq, n_sel, dim = q.shape
    _, hkv, n_keys, _ = k.shape
    host, dev = device_plan.attention_schedule(hq, hkv, dim, q.dtype)
    lib = _native.lib()
    ws_bytes = int(lib.kvr_attention_workspace_bytes(host, len(host), int(hq), int(dim)))
    _native.check(ws_bytes, "kvr_attention_workspace_bytes")
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device) if ws_bytes else None
    strides = _native.i64_array(_native.strides3(q) + _native.strides3(k) + _native.strides3(v)
                                + _native.strides3(out))
    status = lib.kvr_packed_causal_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), device_plan.positions.data_ptr(), int(n_sel),
        int(hq), int(hkv), int(n_keys), int(dim), float(scale), strides, dev.data_ptr(), len(host), host,
        workspace.data_ptr() if workspace is not None else None, ws_bytes, _native.DTYPE_CODES[q.dtype],
        _native.stream_handle(q.device))
    _native.check(status, "kvr_packed_causal_attention")


def indexed_kv_scatter_(out_k, out_v, fresh_k, fresh_v, device_plan) -> None:
    """Copy selected K/V rows exactly, preserving every other storage byte.

    ``out_*[0, h, positions[r], :] = fresh_*[0, h, r, :]``. Output K/V storage
    must be independent of each other and of both fresh inputs. Source and
    destination strides may differ; nothing is made contiguous. Valid unique
    positions give one writer per output element (reference
    indexed_attention.py:179-204).
    """
    tensors = (out_k, out_v, fresh_k, fresh_v)
    _validate_tensors(tensors)
    _validate_plan(device_plan, out_k.device)
    _, heads, _, dim = out_k.shape
    if any((t.shape[1], t.shape[3]) != (heads, dim) for t in tensors):
        raise ValueError("scatter K/V head geometry must match")
    if any(t.shape[2] != device_plan.logical_length for t in tensors[:2]):
        raise ValueError("output sequence length must match the plan")
    if any(t.shape[2] != device_plan.selected_count for t in tensors[2:]):
        raise ValueError("fresh sequence length must match selected_count")
    if not device_plan.selected_count:
        return
    storage = [t.untyped_storage().data_ptr() for t in tensors]
    if storage[0] == storage[1] or any(a == b for a in storage[:2] for b in storage[2:]):
        raise ValueError("output K/V storage must be independent of outputs and fresh sources")
    _require_gfx950(out_k.device)
    with torch.cuda.device(out_k.device):
        _scatter_native(out_k, out_v, fresh_k, fresh_v, device_plan.positions, device_plan.selected_count)


def rope_indexed_kv_scatter_(query, query_out, out_k, out_v, fresh_k, fresh_v, cos, sin, device_plan) -> None:
    """Fresh-row epilogue of one layer in one launch: RoPE of the fresh queries
    (into ``query_out``) and keys at their absolute positions, then the keys and
    values scattered into ``out_k``/``out_v`` at the plan's positions.

    query/query_out=[1,Hq,B,D], fresh_k/fresh_v=[1,Hkv,B,D], out_k/out_v=
    [1,Hkv,N,D], cos/sin=[1,B,D] (the rotary embedding of the selected
    positions, in the tensors' dtype). Bit-identical to the native
    ``apply_rotary_pos_emb`` (transformers 5.15.0 modeling_llama.py:137-160)
    followed by ``indexed_kv_scatter_`` (reference indexed_attention.py:179-204);
    the reference runs these as separate eager ops. Every other storage byte of
    the outputs is preserved.
    """
    tensors = (query, query_out, out_k, out_v, fresh_k, fresh_v)
    _validate_tensors(tensors, dtypes=_NATIVE_DTYPES, dims=None)
    _validate_plan(device_plan, out_k.device)
    _, hq, n_sel, dim = query.shape
    _, hkv, _, _ = out_k.shape
    if dim % 2:
        raise ValueError("rotary head dimension must be even")
    if query_out.shape != query.shape or any(t.shape[1] != hkv or t.shape[3] != dim for t in tensors[2:]):
        raise ValueError("query/KV head geometry must match")
    if any(t.shape[2] != device_plan.logical_length for t in (out_k, out_v)):
        raise ValueError("output sequence length must match the plan")
    if any(t.shape[2] != device_plan.selected_count for t in (query, fresh_k, fresh_v)):
        raise ValueError("fresh sequence length must match selected_count")
    for table in (cos, sin):
        if (not isinstance(table, torch.Tensor) or table.dtype != query.dtype or table.device != query.device
                or table.shape[-2:] != (n_sel, dim) or table.numel() != n_sel * dim or table.stride(-1) <= 0
                or table.stride(-2) < 0):
            raise ValueError("cos/sin must be [1, selected_count, head_dim] in the query dtype and device")
    if not device_plan.selected_count:
        return
    storage = [t.untyped_storage().data_ptr() for t in tensors]
    writes, reads = storage[1:4], [storage[0], *storage[4:], cos.untyped_storage().data_ptr(),
                                   sin.untyped_storage().data_ptr()]
    if len(set(writes)) != 3 or any(w == r for w in writes for r in reads):
        raise ValueError("output query/K/V storage must be independent of each other and of the inputs")
    _require_gfx950(out_k.device)
    with torch.cuda.device(out_k.device):
        _rope_scatter_native(query, query_out, out_k, out_v, fresh_k, fresh_v, cos, sin, device_plan.positions,
                             device_plan.selected_count)


def indexed_causal_attention(q, k, v, device_plan, scale=None):
    """Attend packed queries to their entire absolute causal prefix.

    q=[1,Hq,B,D], k/v=[1,Hkv,N,D], result=[1,Hq,B,D] contiguous. Selected row r
    attends keys j <= positions[r], itself included; K/V must already hold the
    fresh selected rows. Inference only, no dropout. QK^T and PV run on the
    gfx950 bf16/fp16 MFMA with fp32 accumulation; softmax statistics are fp32
    and probabilities enter PV as a hi+lo pair of 16-bit values, so they are
    not rounded to the input dtype (reference indexed_attention.py:207-241).
    """
    _validate_tensors((q, k, v))
    _validate_plan(device_plan, q.device)
    if k.shape != v.shape or q.shape[3] != k.shape[3]:
        raise ValueError("attention K/V shapes and Q/K/V head dimensions must match")
    if q.shape[1] % k.shape[1]:
        raise ValueError("query head count must be divisible by KV head count")
    if q.shape[2] != device_plan.selected_count or k.shape[2] != device_plan.logical_length:
        raise ValueError("attention sequence lengths must match the plan")
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if isinstance(scale, bool) or not isinstance(scale, Real) or not math.isfinite(scale):
        raise ValueError("attention scale must be a finite host real number")
    _require_gfx950(q.device)
    output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if not device_plan.selected_count:
        return output
    with torch.cuda.device(q.device):
        _attention_native(q, k, v, output, device_plan, float(scale))
    return output
