"""GPU parity of the interval writeback (kvr_copy_kv_interval).

Every tensor here is a view made with ``as_strided`` over a flat random
storage, so the expected storage after a copy can be computed independently of
the kernel: a storage-index map (``arange`` viewed with the tensor's strides)
says which storage element each view element is, and the interval rows are
assigned through those maps. The whole storages (holes, padding, rows outside
the interval, the sources) must then match bit for bit, and the copied views
must equal the C oracle's ``orc_copy_interval``.

Vectors from the reference's tests/test_writeback.py: the four layouts (dense,
every other row and dim with offsets, token-major, padded batch and head axes),
the shapes and intervals, the rejected intervals and tensor contracts, and the
fp16/bf16 payloads (signed zeros, infinities, a NaN with payload, a subnormal).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from strided_views import PAYLOADS, host_bits, payload_rows, same_bits, storage_index, strided_over_storage

pytestmark = pytest.mark.gpu

CODE = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16}


CASES = [((1, 8, 37, 128), 3, 4), ((2, 3, 71, 37), 5, 22), ((2, 5, 33, 7), 0, 33), ((1, 1, 9, 13), 0, 0),
         ((1, 8, 300, 128), 17, 289)]
ARRANGEMENTS = {"dense": ("dense",) * 4, "mixed": ("sparse", "token_major", "padded", "sparse")}


@pytest.mark.parametrize("layouts", list(ARRANGEMENTS))
@pytest.mark.parametrize("shape,start,end", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_interval_copy_writes_exactly_the_interval(gpu_device, shape, start, end, dtype, layouts):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    gen = torch.Generator(device=gpu_device).manual_seed(5000 + 7 * end + shape[3])
    src_shape = shape[:2] + (max(1, end), shape[3])
    made = [strided_over_storage(s, dtype, gpu_device, layout, gen)
            for s, layout in zip((shape, shape, src_shape, src_shape), ARRANGEMENTS[layouts])]
    storages, views = [m[0] for m in made], [m[1] for m in made]
    before = [s.clone() for s in storages]
    expected = [s.clone() for s in storages]
    for out, src in ((0, 2), (1, 3)):
        dst_idx = storage_index(views[out])[:, :, start:end, :]
        src_idx = storage_index(views[src])[:, :, start:end, :]
        expected[out][dst_idx.reshape(-1)] = before[src][src_idx.reshape(-1)]
    oracle = [orc.copy_interval(host_bits(views[out]), host_bits(views[src]), start, start, end - start,
                                CODE[dtype]) for out, src in ((0, 2), (1, 3))]

    copy_kv_interval_(*views, start, end)
    torch.cuda.synchronize()
    for actual, want in zip(storages, expected):
        assert same_bits(actual, want)
    assert np.array_equal(host_bits(views[0]), oracle[0]) and np.array_equal(host_bits(views[1]), oracle[1])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_scatter_fresh_kv_writes_fresh_rows_at_the_interval(gpu_device, dtype):
    from kv_cache_repair_amd.kernels.writeback import scatter_fresh_kv

    torch.manual_seed(3)
    out_k = torch.randn(1, 8, 64, 128, device=gpu_device).to(dtype)
    out_v = torch.randn_like(out_k)
    fresh_k = torch.randn(1, 5, 8, 128, device=gpu_device).to(dtype).transpose(1, 2)  # HF token-major layout
    fresh_v = torch.randn(1, 5, 8, 128, device=gpu_device).to(dtype).transpose(1, 2)
    expect_k, expect_v = out_k.clone(), out_v.clone()
    expect_k[:, :, 40:45] = fresh_k
    expect_v[:, :, 40:45] = fresh_v
    scatter_fresh_kv(out_k, out_v, fresh_k, fresh_v, 40, 45)
    assert torch.equal(out_k.view(torch.int16), expect_k.view(torch.int16))
    assert torch.equal(out_v.view(torch.int16), expect_v.view(torch.int16))
    with pytest.raises(RuntimeError, match="cover"):
        scatter_fresh_kv(out_k, out_v, fresh_k, fresh_v, 40, 46)


def four(device, shape=(1, 2, 4, 8)):
    return [torch.zeros(shape, device=device) for _ in range(4)]


BAD_INTERVALS = {"negative start": (-1, 2), "reversed": (2, 1), "past the end": (0, 5), "bool start": (True, 2),
                 "float end": (0, 1.0)}


@pytest.mark.parametrize("why", list(BAD_INTERVALS))
def test_intervals_outside_the_contract_are_refused(gpu_device, why):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    tensors = four(gpu_device)
    start, end = BAD_INTERVALS[why]
    with pytest.raises(ValueError, match="interval"):
        copy_kv_interval_(*tensors, start, end)
    assert all(torch.count_nonzero(t) == 0 for t in tensors)


def _spoil(kind, tensors, device):
    """The four copy_kv_interval_ tensors with one contract violation."""
    out_k, out_v, src_k, src_v = tensors
    spoiled = {
        "source_alias": lambda: (out_k, out_v, out_k.view_as(out_k), src_v),   # a source shares out_k's storage
        "output_alias": lambda: (out_k, out_k.view_as(out_k), src_k, src_v),   # the two outputs share storage
        "dtype": lambda: (out_k, out_v, src_k.double(), src_v),
        "shape": lambda: (out_k, out_v, torch.zeros(1, 3, 4, 8, device=device), src_v),
        "zero_stride": lambda: (torch.zeros(1, 1, 4, 8, device=device).expand(1, 2, 4, 8), out_v, src_k, src_v),
        "overlap": lambda: (out_k.as_strided((1, 2, 4, 8), (64, 1, 1, 1)), out_v, src_k, src_v),
    }
    return spoiled[kind]()


@pytest.mark.parametrize("kind", ["source_alias", "output_alias", "dtype", "shape", "zero_stride", "overlap"])
def test_tensors_outside_the_contract_are_refused(gpu_device, kind):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    with pytest.raises(ValueError):
        copy_kv_interval_(*_spoil(kind, four(gpu_device), gpu_device), 0, 2)


@pytest.mark.parametrize("dtype", list(PAYLOADS))
@pytest.mark.parametrize("heads,rows", [(1, 2), (3, 5)])
def test_copied_rows_keep_their_exact_bits(gpu_device, dtype, heads, rows):
    """Special values and NaN payloads survive the copy unchanged (no
    arithmetic, no canonicalisation), in K and V, and rows past the interval
    stay untouched."""
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    bits = payload_rows(dtype, heads, rows, 3, gpu_device)
    src_k = bits.view(dtype)
    src_v = bits.flip(2).contiguous().view(dtype)
    out_k = torch.zeros(1, heads, rows + 2, 3, device=gpu_device, dtype=dtype)
    out_v = torch.zeros_like(out_k)
    copy_kv_interval_(out_k, out_v, src_k, src_v, 0, rows)
    torch.cuda.synchronize()
    assert torch.equal(out_k[:, :, :rows].view(torch.int16), bits)
    assert torch.equal(out_v[:, :, :rows].view(torch.int16), bits.flip(2))
    assert torch.count_nonzero(out_k[:, :, rows:].view(torch.int16)) == 0
    assert torch.count_nonzero(out_v[:, :, rows:].view(torch.int16)) == 0


# ---------------------------------------------------------------------------
# the sequential interval executor (reference execution.py:34-59), whose
# writeback is this kernel
# ---------------------------------------------------------------------------

def _tiny_model(family, dtype, device):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    options = dict(vocab_size=64, hidden_size=64, intermediate_size=96, num_hidden_layers=3, num_attention_heads=4,
                   num_key_value_heads=2, head_dim=16, max_position_embeddings=512, attention_dropout=0.0)
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(41)
        if family == "llama":
            model = LlamaForCausalLM(LlamaConfig(**options))
        else:
            model = Qwen3ForCausalLM(Qwen3Config(**options, layer_types=["full_attention"] * 3))
    model = model.to(device=device, dtype=dtype).eval()
    model.set_attn_implementation("eager")
    return model


# bf16 models run SDPA (the fused kernel): eager attention would multiply bf16
# queries by a transposed key view, a batched product kept off these GPUs
PRECISIONS = [(torch.float32, "eager"), (torch.float32, "sdpa"), (torch.bfloat16, "sdpa")]


@pytest.mark.parametrize("intervals", [[(5, 9)], [(0, 3), (3, 4), (20, 37), (60, 64)], [(63, 64)], []])
@pytest.mark.parametrize("dtype,attn", PRECISIONS)
@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_sequential_executor_equals_the_reference_recurrence_bit_for_bit(gpu_device, family, dtype, attn,
                                                                         intervals):
    """Each interval's forward sees the same prefix values as the reference's
    clone-and-concatenate recurrence (oracle reference_path.sequential_repair),
    so every layer's K/V must match it bit for bit, adjacent intervals included;
    the base cache is never written."""
    from kv_cache_repair_amd.cache import OperatorShim
    from kv_cache_repair_amd.execution import sequential_repair
    from oracle import reference_path as ref

    model = _tiny_model(family, dtype, gpu_device)
    model.set_attn_implementation(attn)
    gen = torch.Generator(device=gpu_device).manual_seed(7)
    ids = torch.randint(0, 64, (1, 64), device=gpu_device, generator=gen)
    with torch.no_grad():
        base = model.base_model(input_ids=ids, use_cache=True).past_key_values
    edited = ids.clone()
    edited[0, ::3] = torch.randint(0, 64, (22,), device=gpu_device, generator=gen)  # rows that change on refresh
    snap = [(l.keys.clone(), l.values.clone()) for l in base.layers]
    out, receipt = sequential_repair(OperatorShim(model), base, edited, intervals)
    expected = ref.sequential_repair(model, base, edited, intervals)
    assert receipt["interval_count"] == len(intervals)
    assert receipt["recomputed_tokens"] == sum(e - s for s, e in intervals)
    assert receipt["conditioned_on_earlier_intervals"] is True
    if not intervals:
        assert out is base
    for got, want, (k0, v0), layer in zip(out.layers, expected.layers, snap, base.layers):
        assert same_bits(got.keys, want.keys) and same_bits(got.values, want.values)
        assert same_bits(layer.keys, k0) and same_bits(layer.values, v0)
        if intervals:
            assert got.keys.data_ptr() != layer.keys.data_ptr()


@pytest.mark.parametrize("intervals", [[(4, 2)], [(0, 5), (4, 8)], [(3, 65)], [(5, 5)], [(-1, 2)]])
def test_sequential_executor_refuses_unordered_or_outside_intervals(gpu_device, intervals):
    from kv_cache_repair_amd.cache import OperatorShim
    from kv_cache_repair_amd.execution import sequential_repair

    model = _tiny_model("llama", torch.float32, gpu_device)
    ids = torch.zeros((1, 64), dtype=torch.long, device=gpu_device)
    with torch.no_grad():
        base = model.base_model(input_ids=ids, use_cache=True).past_key_values
    with pytest.raises(ValueError, match="sorted, disjoint, and within"):
        sequential_repair(OperatorShim(model), base, ids, intervals)


@pytest.mark.parametrize("dtype,attn", PRECISIONS)
@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_oneshot_control_equals_the_reference_packed_schedule(gpu_device, family, dtype, attn):
    """The one-shot control (every selected row in one forward at its absolute
    position) is the packed schedule: against the reference's packed SDPA
    restatement within the packed executor's tolerances; adjacent intervals are
    accepted and coalesced, an empty support returns the base."""
    from kv_cache_repair_amd.cache import OperatorShim
    from kv_cache_repair_amd.execution import oneshot_sparse_repair
    from oracle import reference_path as ref

    model = _tiny_model(family, dtype, gpu_device)
    model.set_attn_implementation(attn)
    gen = torch.Generator(device=gpu_device).manual_seed(13)
    ids = torch.randint(0, 64, (1, 64), device=gpu_device, generator=gen)
    with torch.no_grad():
        base = model.base_model(input_ids=ids, use_cache=True).past_key_values
    edited = ids.clone()
    edited[0, 2::4] = torch.randint(0, 64, (16,), device=gpu_device, generator=gen)
    snap = [(l.keys.clone(), l.values.clone()) for l in base.layers]
    out, receipt = oneshot_sparse_repair(OperatorShim(model), base, edited, [(2, 6), (6, 9), (30, 31), (50, 64)])
    assert receipt["executor"] == "oneshot_sparse_repair" and receipt["recomputed_tokens"] == 22
    assert receipt["interval_count"] == 4 and receipt["absolute_position_ids_used"] is True
    want = ref.packed_sdpa_repair(model, base, edited, [(2, 9), (30, 31), (50, 64)])
    tol = dict(rtol=1e-5, atol=2e-5) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    for got, w, (k0, v0), b in zip(out.layers, want.layers, snap, base.layers):
        torch.testing.assert_close(got.keys, w.keys, **tol)
        torch.testing.assert_close(got.values, w.values, **tol)
        assert same_bits(b.keys, k0) and same_bits(b.values, v0)
    same, receipt = oneshot_sparse_repair(OperatorShim(model), base, edited, [])
    assert same is base and receipt["recomputed_tokens"] == 0
    with pytest.raises(ValueError, match="sorted, disjoint, and within"):
        oneshot_sparse_repair(OperatorShim(model), base, edited, [(5, 9), (8, 10)])
