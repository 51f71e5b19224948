"""Common prefix/suffix alignment of token ids across a context edit.

Host-side integer work feeding the rotate step (the shift and the suffix
starts). Same definitions as the reference (src/kv_cache_repair/alignment.py:6-31).
"""

from __future__ import annotations


def shared_prefix_len(left: list[int], right: list[int]) -> int:
    limit = min(len(left), len(right))
    n = 0
    while n < limit and left[n] == right[n]:
        n += 1
    return n


def shared_suffix_len(left: list[int], right: list[int], prefix_len: int) -> int:
    """Longest common suffix that does not overlap the shared prefix."""
    limit = min(len(left), len(right)) - prefix_len
    n = 0
    while n < limit and left[len(left) - 1 - n] == right[len(right) - 1 - n]:
        n += 1
    return n


def token_alignment(old_ids: list[int], new_ids: list[int]) -> dict[str, int]:
    prefix = shared_prefix_len(old_ids, new_ids)
    suffix = shared_suffix_len(old_ids, new_ids, prefix)
    old_start = len(old_ids) - suffix
    new_start = len(new_ids) - suffix
    return {
        "prefix": prefix,
        "suffix": suffix,
        "old_suffix_start": old_start,
        "new_suffix_start": new_start,
        "mandatory_changed_tokens": len(new_ids) - prefix - suffix,
        "position_shift": new_start - old_start,
    }
