"""Common prefix/suffix alignment of token ids across a context edit.

Host-side integer work feeding the rotate step (the shift and the suffix
starts). Same definitions as the reference (src/kv_cache_repair/alignment.py:6-31).
"""

from __future__ import annotations

import ctypes

import numpy as np


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


_ALIGNMENT_KEYS = ("prefix", "suffix", "old_suffix_start", "new_suffix_start", "mandatory_changed_tokens",
                   "position_shift")


def token_alignment_host(old_ids: np.ndarray, new_ids: np.ndarray, vocab: int | None = None) -> dict[str, int]:
    """token_alignment of two 1-D int64 host arrays in one libkvrepair host call
    (kvr_token_alignment, same definitions), which also requires every id to lie
    in [0, vocab) (nonnegative when ``vocab`` is None): ValueError otherwise."""
    from . import _native

    old_ids = np.ascontiguousarray(old_ids, dtype=np.int64).reshape(-1)
    new_ids = np.ascontiguousarray(new_ids, dtype=np.int64).reshape(-1)
    out = (ctypes.c_int64 * 6)()
    # the arrays stay referenced here for the duration of the call
    status = _native.lib().kvr_token_alignment(old_ids.ctypes.data, old_ids.size, new_ids.ctypes.data,
                                               new_ids.size, 0 if vocab is None else int(vocab), out)
    if status != 0:
        raise ValueError("token ids must lie in [0, vocab_size) of the model's embedding table")
    return dict(zip(_ALIGNMENT_KEYS, out))


def token_alignment_arrays(old_ids: np.ndarray, new_ids: np.ndarray) -> dict[str, int]:
    """token_alignment of two 1-D integer arrays (same definitions, vectorised):
    the shared prefix is the first mismatch of the common-length heads, the
    shared suffix the first mismatch of the reversed tails, capped so it does
    not overlap the prefix."""
    old_ids = np.asarray(old_ids).reshape(-1)
    new_ids = np.asarray(new_ids).reshape(-1)
    limit = min(old_ids.size, new_ids.size)
    diff = np.flatnonzero(old_ids[:limit] != new_ids[:limit])
    prefix = int(diff[0]) if diff.size else limit
    tail = limit - prefix
    if tail:
        rdiff = np.flatnonzero(old_ids[old_ids.size - tail:][::-1] != new_ids[new_ids.size - tail:][::-1])
        suffix = int(rdiff[0]) if rdiff.size else tail
    else:
        suffix = 0
    old_start = int(old_ids.size) - suffix
    new_start = int(new_ids.size) - suffix
    return {
        "prefix": prefix,
        "suffix": suffix,
        "old_suffix_start": old_start,
        "new_suffix_start": new_start,
        "mandatory_changed_tokens": int(new_ids.size) - prefix - suffix,
        "position_shift": new_start - old_start,
    }
