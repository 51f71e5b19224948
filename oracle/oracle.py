"""CPU oracle for the packed refresh path — TEST INFRASTRUCTURE ONLY.

This module is the checker that parity tests compare the HIP kernels against.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product package never does.

It wraps ``liboracle.so`` (``kvr_oracle.c``, built by ``build_oracle.py``)
for numpy arrays. bfloat16/float16 tensors travel as their raw uint16 bits.
Each function names the reference file:line it restates (paths under
``/root/reference/src/kv_cache_repair/``).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
F32, F16, BF16 = 0, 1, 2

_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_vp = ctypes.c_void_p
_lib = None


def lib() -> ctypes.CDLL:
    """Load liboracle.so, building it first when it is missing."""
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            from .build_oracle import build

            build()
        L = ctypes.CDLL(str(path))
        L.orc_rope_cos_sin.argtypes = [_f32p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, _f32p, _f32p]
        L.orc_rope_rotate.argtypes = [ctypes.c_int, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                      ctypes.c_int32, _i64p, _i64p, ctypes.c_int64, _f32p, ctypes.c_float,
                                      _f32p, _f32p]
        L.orc_rope_rotate.restype = ctypes.c_int
        L.orc_index_copy.argtypes = [ctypes.c_int, _vp, _i64p, ctypes.c_int64, _vp, _i64p, _i64p, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int32]
        L.orc_copy_interval.argtypes = [ctypes.c_int, _vp, _i64p, _vp, _i64p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64]
        L.orc_attention_f64.argtypes = [ctypes.c_int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _i64p, ctypes.c_int64,
                                        ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                        ctypes.c_double, _f64p]
        L.orc_plan_tiles.argtypes = [_i64p, ctypes.c_int64, _i64p, _i64p]
        L.orc_plan_tiles.restype = ctypes.c_int64
        L.orc_token_alignment.argtypes = [_i64p, ctypes.c_int64, _i64p, ctypes.c_int64, _i64p]
        L.orc_positions_to_intervals.argtypes = [_i64p, ctypes.c_int64, _i64p]
        L.orc_positions_to_intervals.restype = ctypes.c_int64
        for name in ("orc_f32_to_bf16", "orc_f32_to_f16"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_uint16
        for name in ("orc_bf16_to_f32", "orc_f16_to_f32"):
            getattr(L, name).argtypes = [ctypes.c_uint16]
            getattr(L, name).restype = ctypes.c_float
        _lib = L
    return _lib


def _ptr(a: np.ndarray, kind=_vp):
    return a.ctypes.data_as(kind) if kind is not _vp else ctypes.c_void_p(a.ctypes.data)


def _strides(a: np.ndarray) -> np.ndarray:
    return np.array([s // a.itemsize for s in a.strides], dtype=np.int64)


def _check3(a: np.ndarray, dtype: int):
    expect = np.float32 if dtype == F32 else np.uint16
    if a.dtype != expect or a.ndim != 3:
        raise ValueError(f"oracle expects rank-3 {expect.__name__} arrays, got {a.dtype} {a.shape}")


def rope_cos_sin(inv_freq: np.ndarray, position: int, scaling: float = 1.0):
    """fp32 cos/sin of inv_freq*position (transformers 5.15.0 modeling_llama.py:113-127)."""
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    c = np.empty(inv.shape[0], np.float32)
    s = np.empty(inv.shape[0], np.float32)
    lib().orc_rope_cos_sin(_ptr(inv, _f32p), inv.shape[0], int(position), float(scaling), _ptr(c, _f32p),
                           _ptr(s, _f32p))
    return c, s


def rope_rotate(key: np.ndarray, dtype: int, shift: int, inv_freq: np.ndarray, *, scaling: float = 1.0,
                rotary_dim: int | None = None, cos_sin: tuple[np.ndarray, np.ndarray] | None = None) -> np.ndarray:
    """shifted_suffix_keys (cache.py:47-77) of a [heads, rows, head_dim] key view.

    ``cos_sin`` optionally supplies the fp32 cos/sin vectors (rotary_dim/2
    entries) instead of the oracle's correctly rounded ones.
    """
    _check3(key, dtype)
    heads, rows, dim = key.shape
    rd = dim if rotary_dim is None else int(rotary_dim)
    out = np.empty((heads, rows, dim), dtype=key.dtype)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    ss, ds = _strides(key), _strides(out)
    cs = sn = None
    if cos_sin is not None:
        cs = np.ascontiguousarray(cos_sin[0], dtype=np.float32)
        sn = np.ascontiguousarray(cos_sin[1], dtype=np.float32)
    rc = lib().orc_rope_rotate(dtype, _ptr(key), _ptr(out), heads, rows, dim, rd, _ptr(ss, _i64p), _ptr(ds, _i64p),
                               int(shift), _ptr(inv, _f32p), float(scaling),
                               _ptr(cs, _f32p) if cs is not None else None,
                               _ptr(sn, _f32p) if sn is not None else None)
    if rc != 0:
        raise ValueError("oracle rope_rotate rejected its arguments")
    return out


def index_copy(out: np.ndarray, fresh: np.ndarray, positions, dtype: int) -> np.ndarray:
    """Return a copy of ``out`` [heads, n_keys, D] with rows ``positions`` taken
    from ``fresh`` [heads, n_sel, D] (packed_cache.py:189-191)."""
    _check3(out, dtype)
    _check3(fresh, dtype)
    result = np.array(out, copy=True)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    rs, fs = _strides(result), _strides(fresh)
    lib().orc_index_copy(dtype, _ptr(result), _ptr(rs, _i64p), result.shape[1], _ptr(fresh), _ptr(fs, _i64p),
                         _ptr(pos, _i64p), pos.shape[0], result.shape[0], result.shape[2])
    return result


def copy_interval(out: np.ndarray, src: np.ndarray, out_start: int, in_start: int, width: int,
                  dtype: int) -> np.ndarray:
    """Return a copy of ``out`` [batch, heads, tokens, D] whose rows
    [out_start, out_start + width) are rows [in_start, ...) of ``src``
    (kernels/writeback.py:18-60; _writeback_triton.py:44-59 with in_start 0)."""
    expect = np.float32 if dtype == F32 else np.uint16
    for a in (out, src):
        if a.ndim != 4 or a.dtype != expect:
            raise ValueError("oracle copy_interval needs 4-D arrays of the dtype's storage type")
    if out.shape[0] != src.shape[0] or out.shape[1] != src.shape[1] or out.shape[3] != src.shape[3]:
        raise ValueError("oracle copy_interval batch/heads/head_dim differ")
    if not (0 <= out_start and out_start + width <= out.shape[2] and 0 <= in_start
            and in_start + width <= src.shape[2]):
        raise ValueError("oracle copy_interval rows out of range")
    result = np.array(out, copy=True)
    lib().orc_copy_interval(dtype, _ptr(result), _ptr(_strides(result), _i64p), _ptr(src),
                            _ptr(_strides(src), _i64p), out.shape[0], out.shape[1], width, out.shape[3], out_start,
                            in_start)
    return result


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, positions, dtype: int,
                  scale: float | None = None) -> np.ndarray:
    """Dense fp64 masked GQA attention (tests/test_indexed_attention.py:106-116).

    q [Hq, B, D], k/v [Hkv, N, D] -> [Hq, B, D] float64.
    """
    for a in (q, k, v):
        _check3(a, dtype)
    hq, b, d = q.shape
    hkv, n, _ = k.shape
    if hq % hkv or v.shape != k.shape or k.shape[2] != d:
        raise ValueError("oracle attention shapes do not agree")
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    out = np.zeros((hq, b, d), np.float64)
    scale = d ** -0.5 if scale is None else float(scale)
    lib().orc_attention_f64(dtype, _ptr(q), _ptr(_strides(q), _i64p), _ptr(k), _ptr(_strides(k), _i64p), _ptr(v),
                            _ptr(_strides(v), _i64p), _ptr(pos, _i64p), b, hq, hkv, n, d, scale,
                            _ptr(out, _f64p))
    return out


def plan_tiles(positions) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """IndexedPlan full_prefix_tiles / total_tiles (indexed_attention.py:75-79)."""
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    n = pos.shape[0]
    full = np.zeros(max(1, (n + 15) // 16), np.int64)
    total = np.zeros_like(full)
    t = lib().orc_plan_tiles(_ptr(pos, _i64p), n, _ptr(full, _i64p), _ptr(total, _i64p))
    return tuple(int(x) for x in full[:t]), tuple(int(x) for x in total[:t])


_ALIGN_KEYS = ("prefix", "suffix", "old_suffix_start", "new_suffix_start", "mandatory_changed_tokens",
               "position_shift")


def token_alignment(old_ids, new_ids) -> dict[str, int]:
    """token_alignment (alignment.py:21-31)."""
    old = np.ascontiguousarray(old_ids, dtype=np.int64)
    new = np.ascontiguousarray(new_ids, dtype=np.int64)
    out = np.zeros(6, np.int64)
    lib().orc_token_alignment(_ptr(old, _i64p), old.shape[0], _ptr(new, _i64p), new.shape[0], _ptr(out, _i64p))
    return {k: int(v) for k, v in zip(_ALIGN_KEYS, out)}


def positions_to_intervals(positions) -> list[tuple[int, int]]:
    """positions_to_intervals (execution.py:14-23)."""
    pos = np.array(positions, dtype=np.int64).reshape(-1)
    out = np.zeros(2 * max(1, pos.shape[0]), np.int64)
    n = lib().orc_positions_to_intervals(_ptr(pos, _i64p), pos.shape[0], _ptr(out, _i64p))
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]


def f32_to_bf16_bits(x: float) -> int:
    return int(lib().orc_f32_to_bf16(float(x)))


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


def bf16_bits_to_f32(b: int) -> float:
    return float(lib().orc_bf16_to_f32(int(b)))


def f16_bits_to_f32(b: int) -> float:
    return float(lib().orc_f16_to_f32(int(b)))


def query_relevance_f64(embed: np.ndarray, ids, query_ids, boost: float = 0.25) -> np.ndarray:
    """dense_query_relevance_scores (scoring.py:11-72) in float64.

    score[t] = max_j <E[ids[t]] / max(|E[ids[t]]|, 1e-12), E[q_j] / max(|E[q_j]|, 1e-12)>
               + boost * [ids[t] in query_ids]
    (F.normalize of each embedding row, the matmul against the normalised query
    rows, max over the query tokens, the exact-id boost). ``embed`` holds the
    table's values as float32/float64 (16-bit tables: their decoded values).
    """
    table = np.asarray(embed, dtype=np.float64)
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    query = np.asarray(query_ids, dtype=np.int64).reshape(-1)
    if query.size == 0:
        raise ValueError("dense query scorer requires query tokens")

    def unit(rows):
        return rows / np.maximum(np.linalg.norm(rows, axis=1, keepdims=True), 1e-12)

    similarity = (unit(table[ids]) @ unit(table[query]).T).max(axis=1)
    return similarity + np.where(np.isin(ids, query), boost, 0.0)
