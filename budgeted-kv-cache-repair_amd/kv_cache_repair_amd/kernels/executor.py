"""Cache and interval validators of the packed executor contract.

Same acceptance rules and error class as the reference validators
(src/kv_cache_repair/kernels/executor.py:19-47 and :50-70), re-derived for the
transformers 5.15 cache, which exposes layers as ``cache.layers[i].keys/.values``.
"""

from __future__ import annotations

from numbers import Integral
from typing import Any, Sequence

import torch


def layer_kv(cache: Any, index: int):
    """(keys, values) of one cache layer."""
    layer = cache.layers[index]
    return layer.keys, layer.values


def tensor_layout():
    """The _kvr_layout extension (built in-tree with libkvrepair.so): every
    cache layer's K/V layout and addresses in one pass over torch's tensor
    metadata. No Python fallback: a missing build raises here."""
    try:
        from .. import _kvr_layout
    except ImportError as error:
        raise ImportError("kv_cache_repair_amd._kvr_layout is not built: run build_lib.py (or "
                          "__graft_entry__.build())") from error
    return _kvr_layout


def uniform_layers(layers):
    """(K address bytes, V address bytes, first K) when every layer's K and V are
    tensors of one layout (shape, strides, dtype, device), else None; a layer
    without .keys / .values gives None too."""
    try:
        k_raw, v_raw, first, uniform = tensor_layout().kv_layers(layers)
    except AttributeError:
        return None
    return (k_raw, v_raw, first) if uniform else None


def _validate_cache(cache: Any, logical_length: int) -> int:
    layers = getattr(cache, "layers", None)
    if layers is None:
        raise ValueError("base_cache must expose indexed K/V layers")
    layer_count = len(layers)
    if layer_count == 0:
        raise ValueError("base_cache must contain at least one K/V layer")
    # Fast paths: every layer's K and V share one layout (read in one pass), or
    # one shape, dtype and GPU, that satisfies the per-layer checks below;
    # otherwise those checks name the layer.
    same = uniform_layers(layers)
    if same is not None:
        first = same[2]
        if (first.ndim == 4 and first.get_device() >= 0 and first.shape[0] == 1 and first.shape[2] == logical_length
                and first.shape[1] > 0 and first.shape[3] > 0 and first.is_floating_point()):
            return layer_count
    try:
        tensors = [t for entry in layers for t in (entry.keys, entry.values)]
    except AttributeError:
        tensors = None
    if tensors and all(isinstance(t, torch.Tensor) for t in tensors):
        first = tensors[0]
        sig = (first.shape, first.dtype, first.get_device())
        if (first.ndim == 4 and sig[2] >= 0 and first.shape[0] == 1 and first.shape[2] == logical_length
                and first.shape[1] > 0 and first.shape[3] > 0 and first.is_floating_point()
                and all((t.shape, t.dtype, t.get_device()) == sig for t in tensors)):
            return layer_count
    expected_shape = expected_dtype = None
    for layer in range(layer_count):
        try:
            key, value = layer_kv(cache, layer)
        except AttributeError as exc:
            raise ValueError(f"cache layer {layer} must contain one K/V pair") from exc
        if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
            raise ValueError(f"cache layer {layer} K/V must be tensors")
        if key.ndim != 4 or value.ndim != 4:
            raise ValueError(f"cache layer {layer} K/V must have rank four")
        if key.shape != value.shape or key.dtype != value.dtype or key.device != value.device:
            raise ValueError(f"cache layer {layer} K/V geometry, dtype, and device must agree")
        if key.shape[0] != 1 or key.shape[2] != logical_length:
            raise ValueError(f"cache layer {layer} must match the single-batch edited token length")
        if key.shape[1] <= 0 or key.shape[3] <= 0 or not key.is_floating_point():
            raise ValueError(f"cache layer {layer} requires nonempty floating-point KV heads")
        if expected_shape is None:
            expected_shape, expected_dtype = key.shape, key.dtype
        elif key.shape != expected_shape or key.dtype != expected_dtype:
            raise ValueError("cache layers must have regular shapes and matching dtypes")
    return layer_count


def _validate_intervals(intervals: Sequence[tuple[int, int]], logical_length: int) -> tuple[tuple[int, int], ...]:
    if not isinstance(intervals, (list, tuple)):
        raise ValueError("intervals must be a list or tuple of maximal half-open ranges")
    result = []
    previous_end = -1
    for interval in intervals:
        # fast path: a (start, end) tuple of plain ints (what every caller builds)
        if type(interval) is tuple and len(interval) == 2 and type(interval[0]) is int and type(interval[1]) is int:
            start, end = interval
            if not 0 <= start < end <= logical_length:
                raise ValueError("interval bounds must satisfy 0 <= start < end <= token length")
            if start <= previous_end:
                raise ValueError("intervals must be sorted, disjoint, and maximal (no adjacent ranges)")
            result.append(interval)
            previous_end = end
            continue
        if not isinstance(interval, (tuple, list)) or len(interval) != 2:
            raise ValueError("each interval must contain exactly a start and end")
        if any(isinstance(value, bool) or not isinstance(value, Integral) for value in interval):
            raise ValueError("interval bounds must be integers, not booleans")
        start, end = int(interval[0]), int(interval[1])
        if not 0 <= start < end <= logical_length:
            raise ValueError("interval bounds must satisfy 0 <= start < end <= token length")
        if start <= previous_end:
            raise ValueError("intervals must be sorted, disjoint, and maximal (no adjacent ranges)")
        result.append((start, end))
        previous_end = end
    return tuple(result)
