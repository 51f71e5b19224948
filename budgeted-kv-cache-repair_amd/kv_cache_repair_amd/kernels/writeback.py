"""Interval writeback of fresh K/V rows (libkvrepair kvr_copy_kv_interval).

Same public contract as the reference's writeback module
(src/kv_cache_repair/kernels/writeback.py:6-60): ``copy_kv_interval_`` is a pure
bit copy of rows [start, end) between four [batch, kv_head, token, head_dim]
tensors with arbitrary positive non-overlapping strides, validated before any
device work (same ValueError messages), with no CPU fallback;
``scatter_fresh_kv`` is the executors' trusted launch whose fresh rows [0, W)
land at [start, end) (_writeback_triton.py:44-59).
"""

from __future__ import annotations

import torch

from .. import _native

_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _nonoverlapping_layout(tensor) -> bool:
    """True when no two elements of ``tensor`` share an address.

    Sufficient test for contiguous, permuted and strided slices (the contract
    of src/kv_cache_repair/kernels/writeback.py:6-15): visiting dimensions by
    increasing stride, each stride must clear the extent of the smaller ones.
    Unusual layouts are rejected rather than risking concurrent stores.
    """
    extent = 1
    for stride, size in sorted(zip(tensor.stride(), tensor.shape)):
        if size > 1:
            if stride < extent:
                return False
            extent += (size - 1) * stride
    return True


def _launch(out_key, out_value, new_key, new_value, out_start: int, in_start: int, width: int) -> None:
    batch, heads, _, dim = out_key.shape
    strides = _native.i64_array([int(s) for t in (out_key, out_value, new_key, new_value) for s in t.stride()])
    status = _native.lib().kvr_copy_kv_interval(
        out_key.data_ptr(), out_value.data_ptr(), new_key.data_ptr(), new_value.data_ptr(), batch, heads, width, dim,
        out_start, in_start, strides, _native.DTYPE_CODES[out_key.dtype], _native.stream_handle(out_key.device))
    _native.check(status, "kvr_copy_kv_interval")


def copy_kv_interval_(out_key, out_value, new_key, new_value, start, end) -> None:
    """Overwrite rows [start, end) of two independent GPU output tensors with the
    same rows of two source tensors (source lengths may differ from the outputs').
    Pure copy: no RoPE, arithmetic or attention."""
    tensors = (out_key, out_value, new_key, new_value)
    if any(not isinstance(t, torch.Tensor) or t.ndim != 4 for t in tensors):
        raise ValueError("K/V tensors must have four dimensions")
    if any(t.device != out_key.device or not t.is_cuda for t in tensors):
        raise ValueError("K/V tensors must be on the same CUDA device")
    if out_key.dtype not in _DTYPES:
        raise ValueError("supported dtypes are float16, bfloat16, float32")
    if any(t.dtype != out_key.dtype for t in tensors):
        raise ValueError("K/V dtypes must match")
    if any(type(p) is not int for p in (start, end)):
        raise ValueError("interval bounds must be integers")
    if not 0 <= start <= end <= min(t.shape[2] for t in tensors):
        raise ValueError("interval exceeds a K/V sequence length")
    batch, heads, _, dim = out_key.shape
    if not batch or not heads or not dim:
        raise ValueError("batch, heads, and head dimension must be positive")
    if any((t.shape[0], t.shape[1], t.shape[3]) != (batch, heads, dim) for t in tensors):
        raise ValueError("K/V batch, head count, and head dimensions must match")
    if any(any(s <= 0 for s in t.stride()) for t in tensors):
        raise ValueError("K/V strides must be positive")
    if not all(_nonoverlapping_layout(t) for t in tensors):
        raise ValueError("K/V layouts must be provably nonoverlapping")
    storage = [t.untyped_storage().data_ptr() for t in tensors]
    if any(dst == src for dst in storage[:2] for src in storage[2:]):
        raise ValueError("source and output storage must be separate")
    if storage[0] == storage[1]:
        raise ValueError("output K and V storage must be separate")
    if start == end:
        return
    _launch(out_key, out_value, new_key, new_value, start, start, end - start)


def scatter_fresh_kv(out_key, out_value, new_key, new_value, start: int, end: int) -> None:
    """Trusted launch of the interval executors: fresh rows [0, end - start) of
    ``new_key``/``new_value`` overwrite rows [start, end). The caller has
    qualified the (independently owned) outputs and checked each projection's
    shape, dtype and device; only the launch geometry is checked here."""
    width = end - start
    if width < 0 or new_key.shape[2] < width or new_value.shape[2] < width or end > out_key.shape[2]:
        raise RuntimeError("fresh K/V rows do not cover the interval")
    if width:
        _launch(out_key, out_value, new_key, new_value, start, 0, width)
