"""Support-set helpers and the sequential interval executor.

``positions_to_intervals`` and ``sequential_repair`` keep the reference's
names and contract (src/kv_cache_repair/execution.py:14-59).
"""

from __future__ import annotations

import time
from typing import Any

import torch

from .cache import cache_from_tensors, clone_cache, run_tokens_from_prefix
from .kernels.executor import _validate_cache, layer_kv
from .kernels.writeback import scatter_fresh_kv


def positions_to_intervals(positions: list[int]) -> list[tuple[int, int]]:
    """Coalesce positions (any order, duplicates allowed) into sorted maximal
    half-open runs (reference src/kv_cache_repair/execution.py:14-23)."""
    runs: list[list[int]] = []
    for p in sorted({int(x) for x in positions}):
        if runs and runs[-1][1] == p:
            runs[-1][1] = p + 1
        else:
            runs.append([p, p + 1])
    return [(start, end) for start, end in runs]


def _validate_sequential_intervals(intervals, length: int) -> list[tuple[int, int]]:
    """Sorted, disjoint, non-empty ranges inside [0, length); adjacent ranges are
    allowed (reference execution.py:26-31)."""
    out = []
    previous_end = 0
    for start, end in intervals:
        start, end = int(start), int(end)
        if not previous_end <= start < end <= length:
            raise ValueError("intervals must be sorted, disjoint, and within the edited sequence")
        out.append((start, end))
        previous_end = end
    return out


def _refresh_intervals_(shim: Any, cache: Any, edited_ids_t: torch.Tensor, intervals) -> None:
    """The interval recurrence IN PLACE on a cache the caller owns.

    Interval [s, e) runs the model's own forward over its tokens after a view of
    the cache's first s rows (the forward's cache update concatenates into new
    tensors, so the view is only read), then its fresh K/V rows are copied over
    rows [s, e) of every layer by kvr_copy_kv_interval (a bit copy), so the next
    interval attends to them.
    """
    layers = [layer_kv(cache, i) for i in range(len(cache.layers))]
    for start, end in intervals:
        prefix = cache_from_tensors([(k[:, :, :start], v[:, :, :start]) for k, v in layers])
        fresh = run_tokens_from_prefix(shim, prefix, edited_ids_t[:, start:end], end)
        for i, (key, value) in enumerate(layers):
            new_key, new_value = layer_kv(fresh, i)
            if (new_key.dtype != key.dtype or new_value.dtype != value.dtype or new_key.device != key.device
                    or new_key.shape[:2] != key.shape[:2] or new_key.shape[3] != key.shape[3]
                    or new_key.shape[2] != end or new_value.shape != new_key.shape):
                raise ValueError(f"recomputed K/V of layer {i} do not match the cache's layout or dtype")
            scatter_fresh_kv(key, value, new_key[:, :, start:end], new_value[:, :, start:end], start, end)


@torch.no_grad()
def sequential_repair(shim: Any, base_cache: Any, edited_ids_t: torch.Tensor,
                      intervals: list[tuple[int, int]]) -> tuple[Any, dict[str, Any]]:
    """Refresh the intervals in order, each conditioned on the rows refreshed
    before it (reference execution.py:34-59 over cache.py:147-192).

    The reference rebuilds every layer per interval (a prefix clone, then a
    concatenation of three pieces); here the output is cloned once, in one
    libkvrepair launch for every layer, and each interval writes only its own
    rows (``_refresh_intervals_``). The base cache is not modified; with no
    interval it is returned as it is, as the reference returns it. ``seconds``
    is host time, as in the reference (GPU work may still be queued).
    """
    length = int(edited_ids_t.shape[1])
    intervals = _validate_sequential_intervals(intervals, length)
    cache = base_cache
    started = time.perf_counter()
    if intervals:
        _validate_cache(base_cache, length)
        cache = clone_cache(base_cache)
        _refresh_intervals_(shim, cache, edited_ids_t, intervals)
    return cache, {
        "executor": "sequential_interval_repair",
        "interval_count": len(intervals),
        "recomputed_tokens": sum(end - start for start, end in intervals),
        "seconds": time.perf_counter() - started,
        "conditioned_on_earlier_intervals": True,
    }


@torch.no_grad()
def oneshot_sparse_repair(shim: Any, base_cache: Any, edited_ids_t: torch.Tensor,
                          intervals: list[tuple[int, int]]) -> tuple[Any, dict[str, Any]]:
    """One forward over every selected position at its absolute position
    (reference execution.py:62-140, the control schedule of its benchmark).

    Every selected row attends causally to the cache in which all selected rows
    of that layer are already refreshed; the reference gets this schedule from a
    StaticCache written at absolute cache positions. It is the packed
    executor's schedule, so it runs on that path (libkvrepair attention and
    scatter): adjacent intervals, which the reference accepts here, are
    coalesced into the packed executor's maximal runs first. The base cache is
    not modified; with no interval it is returned as it is.
    """
    from .kernels.packed_cache import packed_interval_repair

    length = int(edited_ids_t.shape[1])
    intervals = _validate_sequential_intervals(intervals, length)
    positions = [p for start, end in intervals for p in range(start, end)]
    started = time.perf_counter()
    if not positions:
        return base_cache, {"executor": "oneshot_sparse_repair", "interval_count": 0, "recomputed_tokens": 0,
                            "seconds": 0.0}
    output, _ = packed_interval_repair(shim, base_cache, edited_ids_t, positions_to_intervals(positions))
    return output, {
        "executor": "oneshot_sparse_repair",
        "interval_count": len(intervals),
        "recomputed_tokens": len(positions),
        "rows_written": len(positions),
        "seconds": time.perf_counter() - started,
        "absolute_position_ids_used": True,
    }
