"""Host-side contract of the packed path, on the CPU (no GPU, no launch).

The validators, the plan and the public entry points must refuse every
request outside the contract before any device work, exactly where the
reference refuses it. Vectors are the reference's own:
IndexedPlan (tests/test_indexed_attention.py:18-62), interval and cache
validation plus the fail-closed model contract (tests/test_packed_cache.py:
162-174, 255-288), positions_to_intervals (tests/test_cache.py:161-162) and the
public API's argument checks (tests/test_api.py:101-149, 251-343). Each
package function is compared with the C oracle's copy where one exists.
"""

from __future__ import annotations

import math
import random
from dataclasses import FrozenInstanceError

import pytest
import torch

from kv_cache_repair_amd import repair_after_deletion, repair_with_positions, select_support
from kv_cache_repair_amd.execution import positions_to_intervals
from kv_cache_repair_amd.kernels import packed_cache
from kv_cache_repair_amd.kernels.executor import _validate_cache, _validate_intervals
from kv_cache_repair_amd.kernels.indexed_attention import (BLOCK_M, BLOCK_N, IndexedPlan, indexed_causal_attention,
                                                           indexed_kv_scatter_)
from kv_cache_repair_amd.cache import OperatorShim, cache_from_tensors
from oracle import oracle as orc


# ----------------------------------------------------------------------------- IndexedPlan
def test_plan_tile_bounds_known_answer_and_ownership():
    source = [3, 4, 8, 9]
    plan = IndexedPlan(source, 10)
    source[1] = 7  # the plan keeps its own immutable copy
    assert (plan.positions, plan.logical_length, plan.selected_count) == ((3, 4, 8, 9), 10, 4)
    assert (plan.full_prefix_tiles, plan.total_tiles) == ((0,), (1,))
    assert (plan.full_prefix_tiles, plan.total_tiles) == orc.plan_tiles(plan.positions)
    with pytest.raises(FrozenInstanceError):
        plan.positions = (1,)


@pytest.mark.parametrize("count", [0, 1, 15, 16, 17, 64])
def test_plan_tile_bounds_bracket_each_16_row_tile(count):
    """Tile t's first key block holds its first row's causal end and its last
    block the last row's: full*64 <= min+1 < (full+1)*64, (total-1)*64 < max+1 <= total*64."""
    positions = [63 + 67 * i for i in range(count)]
    plan = IndexedPlan(positions, 5000)
    tiles = [positions[i:i + BLOCK_M] for i in range(0, count, BLOCK_M)]
    assert len(plan.full_prefix_tiles) == len(plan.total_tiles) == len(tiles)
    for rows, full, total in zip(tiles, plan.full_prefix_tiles, plan.total_tiles):
        assert full * BLOCK_N <= rows[0] + 1 < (full + 1) * BLOCK_N
        assert (total - 1) * BLOCK_N < rows[-1] + 1 <= total * BLOCK_N
    assert (plan.full_prefix_tiles, plan.total_tiles) == orc.plan_tiles(positions)


@pytest.mark.parametrize("positions,length", [
    ([2, 1], 4), ([1, 1], 4), ([-1], 4), ([4], 4), ([True], 4), ([1.0], 4), (torch.tensor([1]), 4),
    ([0], -1), ([], True), ([], 4.0), ([], 1 << 63), (None, 4)])
def test_invalid_plans_are_refused_on_the_host(positions, length):
    with pytest.raises(ValueError):
        IndexedPlan(positions, length)


def test_plan_upload_refuses_a_cpu_target():
    with pytest.raises(ValueError, match="CUDA"):
        IndexedPlan([0], 1).to("cpu")


def test_operators_refuse_cpu_tensors_without_fallback():
    x = torch.zeros((1, 1, 1, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA"):
        indexed_causal_attention(x, x, x, IndexedPlan([0], 1))
    with pytest.raises(ValueError, match="CUDA"):
        indexed_kv_scatter_(x, x, x, x, IndexedPlan([0], 1))


# ----------------------------------------------------------------------------- intervals and positions
def test_positions_to_intervals_known_answer():
    assert positions_to_intervals([5, 2, 3, 2, 8, 6]) == [(2, 4), (5, 7), (8, 9)]
    assert positions_to_intervals([]) == []


def test_positions_to_intervals_matches_the_oracle():
    rng = random.Random(11)
    for _ in range(300):
        positions = [rng.randrange(40) for _ in range(rng.randrange(25))]
        want = orc.positions_to_intervals(sorted(set(positions)))
        assert positions_to_intervals(positions) == [tuple(r) for r in want]
        # maximal runs: each covers consecutive positions and neighbours are separated by a gap
        got = positions_to_intervals(positions)
        assert [p for s, e in got for p in range(s, e)] == sorted(set(positions))
        assert all(a[1] < b[0] for a, b in zip(got, got[1:]))


@pytest.mark.parametrize("intervals", [
    [(3, 5), (5, 6)],          # adjacent: not maximal
    [(5, 6), (3, 4)],          # unsorted
    [(3, 6), (4, 8)],          # overlapping
    [(2, 2)], [(4, 3)],        # empty / reversed
    [(-1, 2)], [(9, 11)],      # outside [0, length)
    [(True, 2)], [(0, 2.0)],   # booleans and floats are not integer bounds
    [(1, 2, 3)], [5], "ab", None])
def test_interval_validation_refuses_non_maximal_or_malformed_sets(intervals):
    with pytest.raises(ValueError):
        _validate_intervals(intervals, 10)


def test_interval_validation_accepts_sorted_separated_runs():
    assert _validate_intervals([(0, 1), (3, 5), (9, 10)], 10) == ((0, 1), (3, 5), (9, 10))
    assert _validate_intervals([], 10) == ()
    assert _validate_intervals(((2, 4),), 10) == ((2, 4),)


def _cache(shapes, dtype=torch.float32):
    return cache_from_tensors([(torch.zeros(s, dtype=dtype), torch.zeros(s, dtype=dtype)) for s in shapes])


@pytest.mark.parametrize("problem", ["no_layers", "rank", "length", "batch", "heads", "kv_mismatch", "integer",
                                     "irregular", "mixed_dtype", "not_a_cache"])
def test_cache_validation_refuses_irregular_caches(problem):
    good = (1, 2, 12, 8)
    cache = {
        "no_layers": lambda: _cache([]),
        "rank": lambda: cache_from_tensors([(torch.zeros(2, 12, 8), torch.zeros(2, 12, 8))]),
        "length": lambda: _cache([(1, 2, 11, 8)]),
        "batch": lambda: _cache([(2, 2, 12, 8)]),
        "heads": lambda: _cache([(1, 0, 12, 8)]),
        "kv_mismatch": lambda: cache_from_tensors([(torch.zeros(good), torch.zeros(1, 2, 12, 16))]),
        "integer": lambda: _cache([good], torch.int32),
        "irregular": lambda: _cache([good, (1, 4, 12, 8)]),
        "mixed_dtype": lambda: cache_from_tensors([(torch.zeros(good), torch.zeros(good)),
                                                   (torch.zeros(good, dtype=torch.float16),
                                                    torch.zeros(good, dtype=torch.float16))]),
        "not_a_cache": lambda: object(),
    }[problem]()
    with pytest.raises(ValueError):
        _validate_cache(cache, 12)


def test_cache_validation_accepts_regular_layers():
    assert _validate_cache(_cache([(1, 2, 12, 8)] * 3), 12) == 3


# ----------------------------------------------------------------------------- packed executor contract
def _model(family="llama", layers=2):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    options = dict(vocab_size=97, hidden_size=32, intermediate_size=64, num_hidden_layers=layers,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=8, max_position_embeddings=128)
    torch.manual_seed(71)
    if family == "llama":
        model = LlamaForCausalLM(LlamaConfig(**options))
    else:
        model = Qwen3ForCausalLM(Qwen3Config(**options, layer_types=["full_attention"] * layers))
    return model.eval()


def _request(model, length=12):
    ids = (torch.arange(length) % 60 + 4).unsqueeze(0)
    with torch.no_grad():
        base = model(input_ids=ids, use_cache=True).past_key_values
    return OperatorShim(model), ids, base


def _bits(cache):
    return [(l.keys.clone(), l.values.clone()) for l in cache.layers]


def _unchanged(cache, snapshot):
    return all(torch.equal(l.keys, k) and torch.equal(l.values, v) for l, (k, v) in zip(cache.layers, snapshot))


def test_empty_support_returns_the_base_cache_without_preparing_work(monkeypatch):
    def forbidden(*args, **kwargs):
        raise AssertionError("an empty support must not qualify, plan or run anything")

    monkeypatch.setattr(packed_cache, "_qualify", forbidden)
    monkeypatch.setattr(packed_cache, "_make_native_view", forbidden)
    monkeypatch.setattr(IndexedPlan, "to", forbidden)
    base = _cache([(1, 2, 0, 8)] * 2)
    out, receipt = packed_cache.packed_interval_repair(object(), base, torch.empty((1, 0), dtype=torch.long), [])
    assert out is base
    assert receipt["output_cache_ownership"] == "borrowed_base" and receipt["recomputed_tokens"] == 0
    receipt = packed_cache.packed_refresh_owned_(object(), base, torch.empty((1, 0), dtype=torch.long), [])
    assert receipt["recomputed_tokens"] == 0


FAULTS = {
    "version": ("transformers", "__version__"),
    "class": None, "base_forward": None, "training": None, "rope": None, "sliding": None,
    "attention_backend": None, "writeback_backend": None, "interval": None, "triton_attention": None,
    "triton_writeback": None, "flex_attention": None, "cpu_device": None,
}


@pytest.mark.parametrize("fault", sorted(FAULTS))
def test_packed_executor_fails_closed_before_device_work(monkeypatch, fault):
    """Every request outside the inspected contract raises ValueError on the host
    and leaves the borrowed base cache bit-identical (reference
    tests/test_packed_cache.py:255-288). A CPU model reaches the device check
    only when nothing else is wrong ("cpu_device")."""
    from transformers import LlamaForCausalLM

    model = _model()
    shim, ids, base = _request(model)
    snapshot = _bits(base)
    kwargs, intervals, match = {}, [(3, 5)], None
    if fault == "version":
        monkeypatch.setattr(packed_cache.transformers, "__version__", "unsupported")
        match = "transformers"
    elif fault == "class":
        class CustomLlama(LlamaForCausalLM):
            pass
        model.__class__ = CustomLlama
        match = "exact native"
    elif fault == "base_forward":
        monkeypatch.setattr(model.model, "forward", lambda **kw: None)
        match = "forward override"
    elif fault == "training":
        model.train()
        match = "eval mode"
    elif fault == "rope":
        model.config.rope_parameters = {"rope_type": "dynamic", "factor": 2.0, "rope_theta": 10000.0}
        match = "RoPE"
    elif fault == "sliding":
        model.config.layer_types = ["full_attention", "sliding_attention"]
        match = "sliding"
    elif fault == "attention_backend":
        kwargs["attention_backend"] = "unknown"
        match = "attention_backend"
    elif fault == "writeback_backend":
        kwargs["writeback_backend"] = "unknown"
        match = "writeback_backend"
    elif fault == "interval":
        intervals = [(3, 5), (5, 6)]
        match = "maximal"
    elif fault == "triton_attention":
        kwargs["attention_backend"] = "triton"
        match = "attention_backend"
    elif fault == "triton_writeback":
        kwargs["writeback_backend"] = "triton"
        match = "writeback_backend"
    elif fault == "flex_attention":
        kwargs["attention_backend"] = "flex"
        match = "attention_backend"
    else:
        match = "ROCm GPU"
    with pytest.raises(ValueError, match=match):
        packed_cache.packed_interval_repair(shim, base, ids, intervals, **kwargs)
    assert _unchanged(base, snapshot)


def test_reference_default_backend_names_are_accepted():
    """The reference's defaults ("sdpa", "torch") name the one HIP path; a CPU
    model then stops only at the device check."""
    assert packed_cache._check_backends("sdpa", "torch") == ("hip", "hip")
    assert packed_cache._check_backends("hip", "hip") == ("hip", "hip")
    model = _model()
    shim, ids, base = _request(model)
    with pytest.raises(ValueError, match="ROCm GPU"):
        packed_cache.packed_interval_repair(shim, base, ids, [(3, 5)], attention_backend="sdpa",
                                            writeback_backend="torch")


@pytest.mark.parametrize("plan", ["short", "longer", "other"])
def test_supplied_plan_must_match_the_support(plan):
    model = _model()
    shim, ids, base = _request(model)
    bad = {"short": IndexedPlan((3, 4, 8), 12), "longer": IndexedPlan((3, 4, 8, 9), 13), "other": object()}[plan]
    with pytest.raises(ValueError, match="IndexedPlan"):
        packed_cache.packed_interval_repair(shim, base, ids, [(3, 5), (8, 10)], plan=bad)


# ----------------------------------------------------------------------------- public API
@pytest.fixture
def tokenizer():
    from tokenizers import Tokenizer
    from tokenizers.models import WordLevel
    from tokenizers.pre_tokenizers import WhitespaceSplit
    from transformers import PreTrainedTokenizerFast

    words = ["[UNK]", "prefix", "obsolete", "discard", "alpha", "beta", "gamma", ".", "red", "blue", "redblue"]
    backend = Tokenizer(WordLevel({w: i for i, w in enumerate(words)}, unk_token="[UNK]"))
    backend.pre_tokenizer = WhitespaceSplit()
    return PreTrainedTokenizerFast(tokenizer_object=backend, unk_token="[UNK]")


@pytest.fixture(params=["llama", "qwen3"])
def api_model(request):
    model = _model(request.param)
    model.set_attn_implementation("eager")
    return model


@pytest.mark.parametrize("budget", [-1, 101, math.nan, math.inf, -math.inf, True])
def test_select_support_rejects_invalid_budgets_before_touching_the_model(budget):
    with pytest.raises(ValueError, match="budget_percent"):
        select_support(None, None, "", "", suffix_start=0, budget_percent=budget)
    with pytest.raises(ValueError, match="budget_percent"):
        repair_after_deletion(None, None, None, "alpha", delete_span=(0, 1), query="", budget_percent=budget)


@pytest.mark.parametrize("delete_span", [None, 7, (0, 0), (-1, 2), (0, 99), (True, 2), (0, 1.5), (0,), (2, 1)])
def test_repair_rejects_invalid_spans_before_touching_the_model(delete_span):
    with pytest.raises(ValueError, match="delete_span"):
        repair_after_deletion(None, None, None, "alpha", delete_span=delete_span, query="alpha")
    with pytest.raises(ValueError, match="delete_span"):
        repair_with_positions(None, None, None, "alpha", delete_span=delete_span, positions=[])


@pytest.mark.parametrize("executor", ["unknown", "direct", "Packed", ""])
def test_repair_rejects_unknown_executors_before_touching_the_model(executor):
    with pytest.raises(ValueError, match="executor"):
        repair_after_deletion(None, None, None, "alpha", delete_span=(0, 1), query="alpha", executor=executor)


@pytest.mark.parametrize("suffix_start", [-1, 2, True, 0.5, "1"])
def test_select_support_rejects_invalid_suffix_boundaries(api_model, tokenizer, suffix_start):
    with pytest.raises(ValueError, match="suffix_start"):
        select_support(api_model, tokenizer, "alpha", "alpha", suffix_start=suffix_start)


@pytest.mark.parametrize("budget,expected", [(0, ()), (100, tuple(range(1, 101)))])
def test_select_support_budget_edges_without_a_forward(api_model, tokenizer, budget, expected):
    text = "prefix " + "alpha beta gamma . " * 25

    def no_forward(module, args):
        raise AssertionError("selection must not run a transformer forward")

    handles = [m.register_forward_pre_hook(no_forward) for m in (api_model, api_model.base_model)]
    try:
        result = select_support(api_model, tokenizer, text, "alpha", suffix_start=1, budget_percent=budget)
    finally:
        for h in handles:
            h.remove()
    assert (result.suffix_start, result.suffix_tokens, result.budget_tokens) == (1, 100, len(expected))
    assert result.positions == expected
    assert [p for s, e in result.intervals for p in range(s, e)] == list(expected)
    assert result.metadata["selection"] == ("shift_only" if budget == 0 else "full_suffix")


def _host_scores(monkeypatch):
    """The oracle's float64 scorer in place of the device scorer (test only: the
    package's scorer has no CPU path)."""
    from kv_cache_repair_amd import api

    def scores(*, model, edited_input_ids, query_token_ids):
        table = model.generator.get_input_embeddings().weight.detach().double().numpy()
        values = orc.query_relevance_f64(table, edited_input_ids[0].numpy(), query_token_ids)
        return [float(v) for v in values], {"exact_token_boost": 0.25}

    monkeypatch.setattr(api, "dense_query_relevance_scores", scores)


@pytest.mark.parametrize("budget,suffix,want", [(2, 100, 2), (5, 100, 5), (2, 3, 1), (5, 3, 1), (50, 3, 2)])
def test_partial_budgets_take_their_ceiling_through_semantic_units(api_model, tokenizer, monkeypatch, budget,
                                                                    suffix, want):
    """ceil(pct/100 * suffix) rows (api.py:77), never rounded to nearest, chosen
    by the semantic-unit allocation (tests/test_api.py:100-149)."""
    _host_scores(monkeypatch)
    text = "prefix " + " ".join(["alpha", "beta", "gamma", "."] * (suffix // 4) + ["alpha"] * (suffix % 4))
    result = select_support(api_model, tokenizer, text, "alpha", suffix_start=1, budget_percent=budget)
    assert (result.suffix_tokens, result.budget_tokens) == (suffix, want)
    assert len(result.positions) == len(set(result.positions)) == want
    assert list(result.positions) == sorted(result.positions) and all(1 <= p <= suffix for p in result.positions)
    assert [p for s, e in result.intervals for p in range(s, e)] == list(result.positions)
    assert result.metadata["selection"] == "sur" and result.metadata["budget_percent"] == budget
    assert result.metadata["allocator"]["budget_tokens"] == want


def test_partial_budgets_on_a_host_model_fail_in_the_device_scorer(api_model, tokenizer):
    """No CPU fallback: the scorer refuses a model that is not on a ROCm device."""
    text = "prefix " + "alpha beta gamma . " * 25
    with pytest.raises(ValueError, match="ROCm GPU device"):
        select_support(api_model, tokenizer, text, "alpha", suffix_start=1, budget_percent=5)


def test_empty_query_is_refused_by_the_selection(api_model, tokenizer, monkeypatch):
    _host_scores(monkeypatch)
    with pytest.raises(ValueError, match="query text tokenization is empty"):
        select_support(api_model, tokenizer, "prefix " + "alpha beta gamma . " * 25, "", suffix_start=1,
                       budget_percent=5)


def test_repair_rejects_training_mode_before_any_device_work(api_model, tokenizer):
    api_model.train()
    with pytest.raises(ValueError, match="model.eval"):
        repair_after_deletion(api_model, tokenizer, None, "prefix alpha", delete_span=(0, 7), query="alpha")


@pytest.mark.parametrize("flag,message", [("quantized", "quantized models"), ("runtime_rope", "default fixed RoPE"),
                                          ("runtime_sliding", "full attention"),
                                          ("forward_override", "per-instance forward overrides"),
                                          ("cpu_device", "ROCm GPU")])
def test_repair_rejects_unsupported_runtime_flags_before_a_forward(api_model, tokenizer, monkeypatch, flag, message):
    if flag == "quantized":
        monkeypatch.setattr(api_model, "is_quantized", True, raising=False)
    elif flag == "runtime_rope":
        monkeypatch.setattr(api_model.base_model.rotary_emb, "rope_type", "dynamic")
    elif flag == "runtime_sliding":
        monkeypatch.setattr(api_model.base_model, "has_sliding_layers", True, raising=False)
    elif flag == "forward_override":
        monkeypatch.setattr(api_model.base_model, "forward", lambda *a, **k: None)

    def no_forward(module, args):
        raise AssertionError("an unsupported runtime must be rejected before a transformer forward")

    handle = api_model.base_model.register_forward_pre_hook(no_forward)
    try:
        with pytest.raises(ValueError, match=message):
            repair_after_deletion(api_model, tokenizer, None, "prefix obsolete alpha", delete_span=(7, 16),
                                  query="alpha", budget_percent=0)
    finally:
        handle.remove()


def test_token_ids_outside_the_vocabulary_are_refused_on_the_host(tokenizer):
    model = _model()
    small = torch.nn.Embedding(5, 32)  # ids of "alpha" (4) fit, "beta" (5) does not
    model.set_input_embeddings(small)
    with pytest.raises(ValueError, match="vocabulary"):
        select_support(model, tokenizer, "alpha beta", "", suffix_start=0, budget_percent=0)
