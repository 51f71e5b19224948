"""Pin the CPU oracle before trusting it as the checker of the HIP kernels.

Each oracle function is checked against the reference's own golden vectors
(cited test file:line under /root/reference/tests), against closed forms and
invariants that a plausible slip (dropped term, swapped half, wrong sign or
index, transposed operand) would break, and against an independent
computation where one exists.
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from oracle import oracle as orc


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage of a CPU tensor as numpy (uint16 for 16-bit floats)."""
    t = t.contiguous()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def from_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.float32:
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


CODE = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16}


# --------------------------------------------------------------------------- conversions
def test_bf16_conversion_matches_torch_rounding_including_ties_and_specials():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10,
                           np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.0e38, 65504.0], np.float32),
                           # exact ties between two bfloat16 values
                           (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    expect = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.f32_to_bf16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, expect)
    assert orc.f32_to_bf16_bits(float("nan")) == 0x7FC0


def test_f16_conversion_matches_torch_rounding_including_subnormals():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 100,
                           rng.standard_normal(500).astype(np.float32) * 1e-6,  # subnormal range
                           np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 6.1035156e-05], np.float32)])
    expect = torch.from_numpy(vals).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, expect)
    back = np.array([orc.f16_bits_to_f32(int(b)) for b in expect], np.float32)
    assert np.array_equal(back, torch.from_numpy(expect.view(np.int16)).view(torch.float16).float().numpy())


# --------------------------------------------------------------------------- rotate
def _inv_freq(dim: int, theta: float) -> np.ndarray:
    # transformers 5.15.0 modeling_llama.py:108 (fp32 pow and divide)
    return (1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))).numpy()


def test_rotate_with_cos0_sin1_is_rotate_half_kat():
    # reference tests/test_cache.py:89-90: rotate_half([1,2,3,4]) == [-3,-4,1,2]
    key = np.array([[[1.0, 2.0, 3.0, 4.0]]], np.float32)
    out = orc.rope_rotate(key, orc.F32, 7, np.ones(2, np.float32),
                          cos_sin=(np.zeros(2, np.float32), np.ones(2, np.float32)))
    assert out.reshape(-1).tolist() == [-3.0, -4.0, 1.0, 2.0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_zero_shift_is_a_bit_copy(dtype):
    # reference cache.py:53-54 (clone), tests/test_cache.py:93-100
    raw = torch.randn(2, 5, 8).to(dtype)
    raw.view(-1)[3] = float("nan")
    raw.view(-1)[4] = -0.0
    out = orc.rope_rotate(bits(raw), CODE[dtype], 0, _inv_freq(8, 10000.0))
    assert same_bits(out, bits(raw))


def test_rotation_matches_closed_form_in_fp64():
    # k' = k cos(s w) + rotate_half(k) sin(s w), w_i = theta^(-2i/D), split halves
    rng = np.random.default_rng(2)
    dim, shift = 16, -37
    inv = _inv_freq(dim, 10000.0)
    key = rng.standard_normal((3, 6, dim)).astype(np.float32)
    out = orc.rope_rotate(key, orc.F32, shift, inv).astype(np.float64)
    ang = (inv.astype(np.float32) * np.float32(shift)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    k = key.astype(np.float64)
    h = dim // 2
    expect = np.concatenate([k[..., :h] * c - k[..., h:] * s, k[..., h:] * c + k[..., :h] * s], axis=-1)
    np.testing.assert_allclose(out, expect, rtol=0, atol=4e-6 * np.abs(k).max())


def test_rotation_composes_and_preserves_pair_norms():
    rng = np.random.default_rng(3)
    dim = 32
    inv = _inv_freq(dim, 500000.0)
    key = rng.standard_normal((2, 9, dim)).astype(np.float32)
    ab = orc.rope_rotate(orc.rope_rotate(key, orc.F32, -11, inv), orc.F32, -29, inv)
    direct = orc.rope_rotate(key, orc.F32, -40, inv)
    np.testing.assert_allclose(ab, direct, atol=2e-5)
    h = dim // 2
    norm = lambda x: x[..., :h] ** 2 + x[..., h:] ** 2  # noqa: E731
    np.testing.assert_allclose(norm(direct), norm(key), rtol=2e-5, atol=1e-6)
    # inverse rotation restores the key
    np.testing.assert_allclose(orc.rope_rotate(direct, orc.F32, 40, inv), key, atol=2e-5)


def test_partial_rotary_passes_tail_dims_through_bitwise():
    # reference cache.py:74-77
    rng = np.random.default_rng(4)
    key = rng.standard_normal((2, 4, 16)).astype(np.float32)
    out = orc.rope_rotate(key, orc.F32, -5, _inv_freq(8, 10000.0), rotary_dim=8)
    assert np.array_equal(out[..., 8:], key[..., 8:])
    full8 = orc.rope_rotate(np.ascontiguousarray(key[..., :8]), orc.F32, -5, _inv_freq(8, 10000.0))
    assert np.array_equal(out[..., :8], full8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shift", [-1, -32, -128, -512, 3])
def test_rotation_matches_the_eager_torch_chain_bitwise(dtype, shift):
    """Same rounding sequence as the reference eager ops (cache.py:62-73), given
    the same fp32 cos/sin: (k*c) and (rotate_half(k)*s) and their sum each
    rounded to the key dtype."""
    from oracle.reference_path import rotate_half

    torch.manual_seed(5)
    dim = 128
    key = torch.randn(1, 4, 33, dim).to(dtype)
    inv = torch.from_numpy(_inv_freq(dim, 500000.0))
    freqs = inv * float(shift)
    emb = torch.cat((freqs, freqs))
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    eager = key * cos + rotate_half(key) * sin
    got = orc.rope_rotate(bits(key[0]), CODE[dtype], shift, inv.numpy(),
                          cos_sin=(freqs.cos().numpy(), freqs.sin().numpy()))
    assert same_bits(got, bits(eager[0]))


def test_oracle_cos_sin_agrees_with_torch_after_cast_to_bfloat16():
    # correctly rounded fp32 cos/sin vs torch's: equal once cast to bfloat16
    inv = _inv_freq(128, 500000.0)
    for shift in (-1, -128, -512, -1024, -4096, 17):
        c, s = orc.rope_cos_sin(inv, shift)
        tc = (torch.from_numpy(inv) * float(shift)).cos()
        ts = (torch.from_numpy(inv) * float(shift)).sin()
        assert np.array_equal(torch.from_numpy(c).to(torch.bfloat16).float().numpy(),
                              tc.to(torch.bfloat16).float().numpy())
        assert np.array_equal(torch.from_numpy(s).to(torch.bfloat16).float().numpy(),
                              ts.to(torch.bfloat16).float().numpy())
        np.testing.assert_allclose(c, tc.numpy(), rtol=0, atol=2.4e-7)


def test_rotation_reproduces_clean_prefill_keys_at_layer_zero():
    """Layer-0 invariant (reference tests/test_cache.py:103-119): layer-0 keys
    depend only on the token and its position, so rotating the old suffix keys
    by the deletion shift gives the clean prefill keys of the edited prompt."""
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(3)
    model = LlamaForCausalLM(LlamaConfig(vocab_size=32, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                                         num_attention_heads=4, num_key_value_heads=2,
                                         max_position_embeddings=64)).eval()
    old_ids = torch.tensor([[1, 2, 9, 10, 3, 4, 5, 6]])
    new_ids = torch.tensor([[1, 2, 3, 4, 5, 6]])
    with torch.no_grad():
        old = model(input_ids=old_ids, use_cache=True).past_key_values
        clean = model(input_ids=new_ids, use_cache=True).past_key_values
    inv = model.model.rotary_emb.inv_freq.numpy()
    old_k0 = old.layers[0].keys[0]
    tail = orc.rope_rotate(bits(old_k0[:, 4:]), orc.F32, -2, inv)
    np.testing.assert_allclose(tail, clean.layers[0].keys[0, :, 2:].numpy(), rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------- scatter
@pytest.mark.parametrize("dtype,payload", [
    (torch.float16, [0, -32768, 31744, -1024, 32257, 1]),   # reference tests/test_indexed_attention.py:286
    (torch.bfloat16, [0, -32768, 32640, -128, 32705, 1]),   # reference tests/test_indexed_attention.py:287
])
def test_scatter_copies_nan_and_signed_zero_payload_bits(dtype, payload):
    raw = np.array(payload, np.int16).view(np.uint16)
    fresh = np.tile(raw, 32).reshape(1, 3, 64)
    out = np.zeros((1, 9, 64), np.uint16)
    got = orc.index_copy(out, fresh, [0, 3, 8], CODE[dtype])
    assert np.array_equal(got[:, [0, 3, 8]], fresh)
    assert not got[:, [1, 2, 4, 5, 6, 7]].any()


def test_scatter_matches_torch_index_copy_on_strided_views():
    torch.manual_seed(6)
    backing = torch.randn(3, 2 * 40 + 3, 2 * 16 + 5)
    out_view = backing[:, 1:1 + 80:2, 2:2 + 32:2]          # "holes" layout
    fresh_backing = torch.randn(9, 3, 16)
    fresh = fresh_backing.transpose(0, 1)                    # token-major view
    positions = [0, 3, 4, 8, 9, 17, 30, 38, 39]
    expect = out_view.clone()
    expect.index_copy_(1, torch.tensor(positions), fresh)
    got = orc.index_copy(out_view.numpy(), fresh.numpy(), positions, orc.F32)
    assert np.array_equal(got, expect.numpy())


def test_scatter_skips_out_of_range_positions():
    out = np.zeros((1, 4, 8), np.float32)
    fresh = np.ones((1, 3, 8), np.float32)
    got = orc.index_copy(out, fresh, [-1, 2, 4], orc.F32)
    assert got[0, 2].tolist() == [1.0] * 8 and got.sum() == 8


# --------------------------------------------------------------------------- interval writeback
@pytest.mark.parametrize("shape,start,end", [((1, 8, 37, 16), 3, 4), ((2, 3, 71, 37), 5, 22),
                                             ((2, 5, 33, 7), 0, 33), ((1, 1, 9, 13), 0, 0)])
def test_copy_interval_matches_slice_assignment_on_strided_views(shape, start, end):
    # shapes and bounds of the reference's tests/test_writeback.py:34-40; torch slice copy is the checker
    torch.manual_seed(701 + end)
    b, h, t, d = shape
    out_backing = torch.randn(b, h, 2 * t + 3, 2 * d + 5)
    out_view = out_backing[:, :, 1:1 + 2 * t:2, 2:2 + 2 * d:2]            # "holes"
    src = torch.randn(b, max(1, end), h, d).permute(0, 2, 1, 3)          # token-major
    expect = out_view.clone()
    expect[:, :, start:end] = src[:, :, start:end]
    got = orc.copy_interval(out_view.numpy(), src.numpy(), start, start, end - start, orc.F32)
    assert np.array_equal(got, expect.numpy())
    fresh = torch.randn(b, h, end - start + 2, d)                        # scatter_fresh_kv: rows [0, W)
    expect = out_view.clone()
    expect[:, :, start:end] = fresh[:, :, :end - start]
    got = orc.copy_interval(out_view.numpy(), fresh.numpy(), start, 0, end - start, orc.F32)
    assert np.array_equal(got, expect.numpy())


@pytest.mark.parametrize("dtype,payload", [
    (torch.float16, [0, -32768, 31744, -1024, 32257, 1]),   # reference tests/test_writeback.py:102-103
    (torch.bfloat16, [0, -32768, 32640, -128, 32705, 1]),
])
def test_copy_interval_keeps_payload_bits(dtype, payload):
    raw = np.array(payload, np.int16).view(np.uint16).reshape(1, 1, 2, 3)
    out = np.zeros((1, 1, 4, 3), np.uint16)
    got = orc.copy_interval(out, raw, 0, 0, 2, CODE[dtype])
    assert np.array_equal(got[:, :, :2], raw) and not got[:, :, 2:].any()


def test_copy_interval_rejects_rows_out_of_range():
    with pytest.raises(ValueError, match="range"):
        orc.copy_interval(np.zeros((1, 1, 4, 3), np.float32), np.zeros((1, 1, 2, 3), np.float32), 3, 0, 2, orc.F32)


def test_writeback_rejects_cpu_tensors_before_any_device_work():
    # reference tests/test_writeback.py:62-65: no silent CPU fallback
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    tensors = [torch.zeros((1, 1, 3, 4)) for _ in range(4)]
    with pytest.raises(ValueError, match="CUDA"):
        copy_kv_interval_(*tensors, 0, 1)


# --------------------------------------------------------------------------- attention
def test_attention_query_at_zero_returns_value_zero():
    # reference tests/test_indexed_attention.py:251-259
    rng = np.random.default_rng(7)
    q = rng.standard_normal((4, 1, 16)).astype(np.float32)
    k = rng.standard_normal((2, 30, 16)).astype(np.float32)
    v = rng.standard_normal((2, 30, 16)).astype(np.float32)
    out = orc.attention_f64(q, k, v, [0], orc.F32)
    np.testing.assert_array_equal(out, np.repeat(v[:, :1].astype(np.float64), 2, axis=0))


def test_attention_arange_values_with_zero_keys_average_to_half_position():
    # reference tests/test_packed_cache.py:207-224: K=0, V=arange -> out = pos/2
    positions = [3, 4, 8, 9]
    q = np.zeros((4, 4, 8), np.float32)
    k = np.zeros((2, 12, 8), np.float32)
    v = np.broadcast_to(np.arange(12, dtype=np.float32)[None, :, None], (2, 12, 8)).copy()
    out = orc.attention_f64(q, k, v, positions, orc.F32)
    for r, p in enumerate(positions):
        np.testing.assert_allclose(out[:, r], p / 2, rtol=0, atol=1e-12)
    # future keys do not matter; a legal unselected past key does
    v2 = v.copy()
    v2[:, 10:] = 10000
    np.testing.assert_array_equal(orc.attention_f64(q, k, v2, positions, orc.F32), out)
    v3 = v.copy()
    v3[:, 1] += 100
    assert (orc.attention_f64(q, k, v3, positions, orc.F32) > out).all()


def test_attention_grouped_query_heads_read_their_kv_head():
    # reference tests/test_indexed_attention.py:208-224
    q = np.zeros((8, 3, 16), np.float32)
    k = np.zeros((2, 131, 16), np.float32)
    v = np.stack([np.full((131, 16), 1.0, np.float32), np.full((131, 16), 2.0, np.float32)])
    out = orc.attention_f64(q, k, v, [0, 64, 130], orc.F32)
    for h in range(8):
        np.testing.assert_allclose(out[h], h // 4 + 1, rtol=0, atol=1e-12)


def test_attention_matches_brute_force_softmax_on_tiny_input():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((2, 2, 4)).astype(np.float32)
    k = rng.standard_normal((1, 5, 4)).astype(np.float32)
    v = rng.standard_normal((1, 5, 4)).astype(np.float32)
    positions, scale = [1, 4], 0.7
    out = orc.attention_f64(q, k, v, positions, orc.F32, scale)
    for h in range(2):
        for r, p in enumerate(positions):
            w = [math.exp(scale * float(np.dot(q[h, r].astype(np.float64), k[0, j].astype(np.float64))))
                 for j in range(p + 1)]
            expect = sum(wj * v[0, j].astype(np.float64) for j, wj in enumerate(w)) / sum(w)
            np.testing.assert_allclose(out[h, r], expect, rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------------------- host integer logic
def test_plan_tile_bounds_kat_and_identities():
    # reference tests/test_indexed_attention.py:18-39
    assert orc.plan_tiles([3, 4, 8, 9]) == ((0,), (1,))
    for count in (0, 1, 15, 16, 17, 64):
        positions = [63 + i * 67 for i in range(count)]
        full, total = orc.plan_tiles(positions)
        assert len(full) == (count + 15) // 16
        for t, start in enumerate(range(0, count, 16)):
            rows = positions[start:start + 16]
            assert full[t] * 64 <= min(rows) + 1 < (full[t] + 1) * 64
            assert (total[t] - 1) * 64 < max(rows) + 1 <= total[t] * 64


@pytest.mark.parametrize("old,new,expect", [
    # reference tests/test_cache.py:43-68
    ([1, 2, 9, 3, 4], [1, 2, 3, 4], (2, 2, 3, 2, 0, -1)),
    ([1, 2], [1, 2], (2, 0, 2, 2, 0, 0)),
    ([1, 2], [], (0, 0, 2, 0, 0, -2)),
    ([1, 2, 3], [1, 8, 9, 3], (1, 1, 2, 3, 2, 1)),
])
def test_alignment_golden_vectors(old, new, expect):
    got = orc.token_alignment(old, new)
    assert tuple(got.values()) == expect


@pytest.mark.parametrize("old,new,expect", [
    ([1, 2, 9, 3, 4], [1, 2, 3, 4], (2, 2, 3, 2, 0, -1)),
    ([1, 2], [1, 2], (2, 0, 2, 2, 0, 0)),
    ([1, 2], [], (0, 0, 2, 0, 0, -2)),
    ([1, 2, 3], [1, 8, 9, 3], (1, 1, 2, 3, 2, 1)),
])
def test_package_alignment_matches_golden_vectors_and_oracle(old, new, expect):
    """The package's list and vectorised alignments against the reference's
    golden tuples (tests/test_cache.py:43-68) and the C oracle on random edits."""
    import numpy as np

    from kv_cache_repair_amd.alignment import token_alignment, token_alignment_arrays, token_alignment_host

    assert tuple(token_alignment(old, new).values()) == expect
    assert tuple(token_alignment_arrays(np.array(old, dtype=np.int64), np.array(new, dtype=np.int64)).values()) == \
        expect
    assert tuple(token_alignment_host(np.array(old, dtype=np.int64), np.array(new, dtype=np.int64), 10).values()) == \
        expect
    rng = random.Random(len(old) * 7 + len(new))
    for _ in range(300):
        base = [rng.randrange(4) for _ in range(rng.randrange(0, 40))]
        a, b = rng.randrange(len(base) + 1), rng.randrange(len(base) + 1)
        a, b = min(a, b), max(a, b)
        edited = base[:a] + [rng.randrange(4) for _ in range(rng.randrange(0, 5))] + base[b:]
        want = orc.token_alignment(base, edited)
        assert token_alignment(base, edited) == want
        assert token_alignment_arrays(np.array(base, dtype=np.int64), np.array(edited, dtype=np.int64)) == want
        assert token_alignment_host(np.array(base, dtype=np.int64), np.array(edited, dtype=np.int64), 4) == want


def test_host_alignment_refuses_ids_outside_the_vocabulary():
    """kvr_token_alignment (the shift-cache build's host call) checks every id of
    both rows against [0, vocab): the build gathers embedding rows by them."""
    import numpy as np

    from kv_cache_repair_amd.alignment import token_alignment_host

    old = np.array([1, 2, 3, 4], dtype=np.int64)
    assert token_alignment_host(old, np.array([1, 3, 4], dtype=np.int64), 5)["position_shift"] == -1
    assert token_alignment_host(old, old, None)["prefix"] == 4  # no vocabulary: ids only nonnegative
    for bad_old, bad_new, vocab in (([1, 2, 5], [1, 2], 5), ([1, 2], [1, 9, 2], 5), ([1, -1], [1], 5),
                                    ([1], [-3], None)):
        with pytest.raises(ValueError, match="vocab"):
            token_alignment_host(np.array(bad_old, dtype=np.int64), np.array(bad_new, dtype=np.int64), vocab)
    # int32 rows are widened; empty rows are valid
    assert token_alignment_host(np.array([7, 8], dtype=np.int32), np.array([], dtype=np.int32), 9)["suffix"] == 0


def test_host_alignment_on_long_rows_matches_the_oracle_and_the_range_rule():
    """Rows long enough for the C scan's 64-id block compares (prefix, suffix and
    the edited middle at every offset relative to the blocks), random deletions,
    insertions and substitutions, against the C oracle's alignment; an id outside
    [0, vocab) planted anywhere in either row is refused."""
    import numpy as np

    from kv_cache_repair_amd.alignment import token_alignment_host

    rng = random.Random(23)
    for trial in range(600):
        base = [rng.randrange(6) for _ in range(rng.randrange(0, 400))]
        edited = list(base)
        for _ in range(rng.randrange(0, 3)):
            at = rng.randrange(len(edited) + 1)
            kind = rng.randrange(3)
            if kind == 0:
                del edited[at:at + rng.randrange(1, 90)]
            elif kind == 1:
                edited[at:at] = [rng.randrange(6) for _ in range(rng.randrange(1, 90))]
            elif edited:
                edited[rng.randrange(len(edited))] = rng.randrange(6)
        if trial % 3 == 0:
            row = base if (trial % 2 and base) or not edited else edited
            if row:
                row[rng.randrange(len(row))] = rng.choice([6, 7, -1, -(1 << 40)])
        bad = any(x < 0 or x >= 6 for x in base + edited)
        if bad:
            with pytest.raises(ValueError, match="vocab"):
                token_alignment_host(np.array(base, dtype=np.int64), np.array(edited, dtype=np.int64), 6)
        else:
            assert token_alignment_host(np.array(base, dtype=np.int64), np.array(edited, dtype=np.int64), 6) == \
                orc.token_alignment(base, edited)


def test_positions_to_intervals_kat_and_brute_force():
    # reference tests/test_cache.py:161-162
    assert orc.positions_to_intervals([5, 2, 3, 2, 8, 6]) == [(2, 4), (5, 7), (8, 9)]
    rng = random.Random(9)
    for _ in range(200):
        pos = [rng.randrange(40) for _ in range(rng.randrange(0, 30))]
        got = orc.positions_to_intervals(pos)
        covered = sorted(p for s, e in got for p in range(s, e))
        assert covered == sorted(set(pos))
        assert all(a[1] < b[0] for a, b in zip(got, got[1:]))  # maximal: gaps between runs


# ---- dense query relevance (scoring.py:11-72) ----
_KAT_TABLE = np.array([[1.0, 0.0], [1.0, 0.0], [-1.0, 0.0], [0.0, 1.0]])


def test_relevance_exact_bonus_applies_only_to_identical_ids_kat():
    # test_scoring.py:16-26: ids [0,1,2,3], query [1] -> [1.0, 1.25, -1.0, 0.0]
    got = orc.query_relevance_f64(_KAT_TABLE, [0, 1, 2, 3], [1])
    assert got.tolist() == pytest.approx([1.0, 1.25, -1.0, 0.0])


def test_relevance_is_preserved_across_the_reference_chunk_boundary_kat():
    # test_scoring.py:29-37: 1024 x id 2 then id 3, query [1, 3] -> [0.0]*1024 + [1.25]
    got = orc.query_relevance_f64(_KAT_TABLE, [2] * 1024 + [3], [1, 3])
    assert got.tolist() == pytest.approx([0.0] * 1024 + [1.25])


def test_relevance_rejects_an_empty_query():
    with pytest.raises(ValueError, match="requires query tokens"):
        orc.query_relevance_f64(_KAT_TABLE, [0], [])


def test_relevance_is_a_max_of_cosines_invariant_to_row_scale():
    rng = np.random.default_rng(11)
    table = rng.standard_normal((50, 24))
    ids = rng.integers(0, 50, 300)
    query = [3, 7, 7, 41]
    base = orc.query_relevance_f64(table, ids, query)
    scaled = orc.query_relevance_f64(table * rng.uniform(0.1, 10.0, (50, 1)), ids, query)
    np.testing.assert_allclose(base, scaled, rtol=0, atol=1e-12)
    # brute force on a few tokens: cosine by the definition, boost by membership
    for t in (0, 17, 299):
        e = table[ids[t]]
        cos = max(float(e @ table[q]) / (np.linalg.norm(e) * np.linalg.norm(table[q])) for q in query)
        assert base[t] == pytest.approx(cos + (0.25 if ids[t] in query else 0.0), abs=1e-12)
    # a zero row normalises to zero (eps clamp): cosine 0
    table[5] = 0.0
    assert orc.query_relevance_f64(table, [5], [3])[0] == 0.0
