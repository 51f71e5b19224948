"""Support-set helpers shared by the API and the executors."""

from __future__ import annotations


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
