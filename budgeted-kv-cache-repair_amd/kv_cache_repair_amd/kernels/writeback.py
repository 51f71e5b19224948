"""Layout proof shared by the operator contracts."""

from __future__ import annotations


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
