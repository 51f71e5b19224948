"""GPU end-to-end parity of the packed refresh executor.

The HIP path (libkvrepair scatter + attention inside the HF 5.15 forward) is
compared with the reference's default packed path (boolean mask, index_copy_,
HF sdpa_attention_forward; restated in oracle/reference_path.py) run on the
same GPU, with the sequential interval recurrence, and with clean prefill,
following the reference tests (tests/test_packed_cache.py).
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def make_model(device, family="llama", kv_heads=2, *, head_dim=8, dtype=torch.float32, seed=71, layers=2):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(seed)
    options = dict(vocab_size=97, hidden_size=4 * head_dim, intermediate_size=8 * head_dim,
                   num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=kv_heads,
                   head_dim=head_dim, max_position_embeddings=512, attention_dropout=0.0)
    if family == "llama":
        model = LlamaForCausalLM(LlamaConfig(**options))
    else:
        model = Qwen3ForCausalLM(Qwen3Config(**options, layer_types=["full_attention"] * layers))
    model.to(device=device, dtype=dtype).eval()
    model.set_attn_implementation("sdpa")
    return model


def make_request(model, length=12):
    from kv_cache_repair_amd.cache import OperatorShim

    ids = (torch.arange(length, device=model.device) % 60 + 4).unsqueeze(0)
    with torch.no_grad():
        base = model(input_ids=ids, use_cache=True).past_key_values
    return OperatorShim(model), ids, base


def snapshot(cache):
    return [(l.keys.clone(), l.values.clone()) for l in cache.layers]


def bits_equal(a, b):
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def assert_ownership_and_untouched(actual, base, snap, intervals):
    selected = {p for s, e in intervals for p in range(s, e)}
    n = base.layers[0].keys.shape[2]
    untouched = [p for p in range(n) if p not in selected]
    for i, layer in enumerate(base.layers):
        assert bits_equal(layer.keys, snap[i][0]) and bits_equal(layer.values, snap[i][1])
        for got, src in ((actual.layers[i].keys, layer.keys), (actual.layers[i].values, layer.values)):
            assert bits_equal(got[:, :, untouched], src[:, :, untouched])
            if selected:
                assert got.untyped_storage().data_ptr() != src.untyped_storage().data_ptr()


def assert_north_star_close(actual, native, control):
    """End-to-end bf16 gate against the reference packed SDPA path (``native``).

    Per-row cosine >= 0.9999, and max-abs <= 2e-2 -- widened to twice the
    reference path's own max-abs error against the fp32 ``control`` where that
    error is larger: refreshed rows of deeper layers carry bf16 rounding from
    every earlier layer, and at K/V magnitudes near 5 (1 bf16 ulp = 0.031) the
    reference path itself sits ~0.06 from fp32, so no second bf16
    implementation can be within 2e-2 of it there.
    """
    a, e, c = actual.float(), native.float(), control.float()
    native_error = (e - c).abs().max().item()
    assert (a - e).abs().max().item() <= max(2e-2, 2.0 * native_error)
    cos = torch.nn.functional.cosine_similarity(a.reshape(-1, a.shape[-1]), e.reshape(-1, e.shape[-1]), dim=-1)
    assert cos.min().item() >= 0.9999


INTERVALS = [[], [(0, 12)], [(2, 12)], [(3, 5), (8, 10)], [(0, 1), (3, 4), (8, 9), (11, 12)]]


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("kv_heads", [1, 2, 4])
@pytest.mark.parametrize("intervals", INTERVALS)
def test_fp32_packed_matches_interval_recurrence_and_reference_sdpa(gpu_device, family, kv_heads, intervals):
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, family, kv_heads)
    shim, ids, base = make_request(model)
    snap = snapshot(base)
    expected = ref.sequential_repair(model, base, ids + 13, intervals)
    reference = ref.packed_sdpa_repair(model, base, ids + 13, intervals)
    actual, receipt = packed_interval_repair(shim, base, ids + 13, intervals)
    for i in range(2):
        for c in (0, 1):
            got = ref.layer_kv(actual, i)[c]
            torch.testing.assert_close(got, ref.layer_kv(expected, i)[c], rtol=1e-5, atol=2e-6)
            torch.testing.assert_close(got, ref.layer_kv(reference, i)[c], rtol=1e-5, atol=2e-6)
    assert_ownership_and_untouched(actual, base, snap, intervals)
    assert receipt["recomputed_tokens"] == sum(e - s for s, e in intervals)
    assert receipt["schedule"] == "packed_selected_rows_layer_major"
    if not intervals:
        assert actual is base
    query = torch.tensor([[77, 78]], device=gpu_device)
    with torch.no_grad():
        got = model(input_ids=query, past_key_values=ref.clone_cache(actual)).logits
        want = model(input_ids=query, past_key_values=ref.clone_cache(expected)).logits
    torch.testing.assert_close(got, want, rtol=1e-5, atol=2e-6)


@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_full_support_matches_clean_prefill(gpu_device, family):
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, family)
    shim, ids, base = make_request(model)
    actual, _ = packed_interval_repair(shim, base, ids + 13, [(0, ids.shape[-1])])
    with torch.no_grad():
        clean = model(input_ids=ids + 13, use_cache=True).past_key_values
    for i in range(2):
        for c in (0, 1):
            torch.testing.assert_close(ref.layer_kv(actual, i)[c], ref.layer_kv(clean, i)[c], rtol=1e-5, atol=2e-6)


def test_supplied_host_plan_matches_exact_support(gpu_device):
    from kv_cache_repair_amd.kernels.indexed_attention import IndexedPlan
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device)
    shim, ids, base = make_request(model)
    intervals = [(3, 5), (8, 10)]
    actual, _ = packed_interval_repair(shim, base, ids + 13, intervals, plan=IndexedPlan((3, 4, 8, 9), 12))
    expected, _ = packed_interval_repair(shim, base, ids + 13, intervals)
    for i in range(2):
        for c in (0, 1):
            assert bits_equal(ref.layer_kv(actual, i)[c], ref.layer_kv(expected, i)[c])
    for invalid in (IndexedPlan((3, 4, 8), 12), IndexedPlan((3, 4, 8, 9), 13), object()):
        with pytest.raises(ValueError, match="IndexedPlan"):
            packed_interval_repair(shim, base, ids, intervals, plan=invalid)


def test_requests_share_no_state_and_leave_native_model_unchanged(gpu_device):
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device)
    model.set_attn_implementation("eager")
    shim, ids, base = make_request(model)
    modules = dict(model.named_modules())
    configs = {n: m.config.to_dict() for n, m in modules.items() if hasattr(m, "config")}
    params = {n: p.data_ptr() for n, p in model.named_parameters()}
    masks = dict(ALL_MASK_ATTENTION_FUNCTIONS)
    with torch.no_grad():
        logits = model(input_ids=ids).logits.clone()
    first, _ = packed_interval_repair(shim, base, ids + 13, [(3, 5), (8, 10)])
    first_snap = snapshot(first)
    second, _ = packed_interval_repair(shim, base, ids + 19, [(0, 2), (10, 12)])
    repeated, _ = packed_interval_repair(shim, base, ids + 13, [(3, 5), (8, 10)])
    for i in range(2):
        assert bits_equal(first.layers[i].keys, first_snap[i][0])
        assert bits_equal(first.layers[i].keys, repeated.layers[i].keys)
        assert bits_equal(first.layers[i].values, repeated.layers[i].values)
    assert first is not second
    assert dict(model.named_modules()) == modules
    assert {n: p.data_ptr() for n, p in model.named_parameters()} == params
    for n, m in model.named_modules():
        if n in configs:
            assert m.config.to_dict() == configs[n]
    assert dict(ALL_MASK_ATTENTION_FUNCTIONS) == masks
    assert "kvr_hip_packed_absolute_attention_v1" in ALL_ATTENTION_FUNCTIONS
    with torch.no_grad():
        assert bits_equal(model(input_ids=ids).logits, logits)


@pytest.mark.parametrize("failure", ["forward_raises", "missing_layer", "replaced_cache"])
def test_failed_transaction_keeps_model_and_base_unchanged(gpu_device, monkeypatch, failure):
    from types import SimpleNamespace

    from transformers.cache_utils import DynamicCache

    import kv_cache_repair_amd.kernels.packed_cache as module

    model = make_model(gpu_device)
    shim, ids, base = make_request(model)
    snap = snapshot(base)

    def failing_forward(**kwargs):
        cache = kwargs["past_key_values"]
        count = kwargs["input_ids"].shape[-1]
        fresh = torch.full((1, 2, count, 8), 999.0, device=gpu_device)
        cache.update(fresh, fresh, 0)
        if failure == "forward_raises":
            raise RuntimeError("injected failure")
        return SimpleNamespace(past_key_values=DynamicCache() if failure == "replaced_cache" else cache)

    monkeypatch.setattr(module, "_make_native_view", lambda base, *args: failing_forward)
    with pytest.raises(RuntimeError):
        module.packed_interval_repair(shim, base, ids + 13, [(3, 5)])
    for i, layer in enumerate(base.layers):
        assert bits_equal(layer.keys, snap[i][0]) and bits_equal(layer.values, snap[i][1])


def assert_within_native_precision_floor(candidate, native_sdpa, matched_fp32):
    """Reference gate (tests/test_packed_cache.py:291-315): the candidate's max-abs
    and RMS error vs an fp32 control are at most twice native SDPA's (fp32 eps floor)."""
    reference = matched_fp32.double()
    candidate, native_sdpa = candidate.double(), native_sdpa.double()
    assert torch.isfinite(candidate).all() and torch.isfinite(native_sdpa).all()
    ce, ne = candidate - reference, native_sdpa - reference
    floor = torch.finfo(torch.float32).eps * max(1.0, reference.abs().max().item())
    for cv, nv in ((ce.abs().max().item(), ne.abs().max().item()),
                   (ce.square().mean().sqrt().item(), ne.square().mean().sqrt().item())):
        assert cv <= 2.0 * max(nv, floor), (cv, nv, floor)


@pytest.mark.parametrize("seed", [71, 191])
@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kv_heads", [1, 2, 4])
def test_low_precision_packed_within_native_sdpa_precision_floor(gpu_device, family, dtype, kv_heads, seed):
    """Reference GPU integration gate (tests/test_packed_cache.py:318-376): length
    137, intervals [(0,1),(3,5),(62,68),(126,132),(136,137)], head_dim 64."""
    from kv_cache_repair_amd.cache import OperatorShim
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, family, kv_heads=kv_heads, head_dim=64, dtype=dtype, seed=seed)
    shim, ids, base = make_request(model, length=137)
    intervals = [(0, 1), (3, 5), (62, 68), (126, 132), (136, 137)]
    positions = torch.tensor([p for s, e in intervals for p in range(s, e)], device=gpu_device)
    snap = snapshot(base)
    control_model = copy.deepcopy(model).float()
    control_base = ref.cache_from_tensors([(l.keys.float(), l.values.float()) for l in base.layers])
    control = ref.packed_sdpa_repair(control_model, control_base, ids + 13, intervals)
    native = ref.packed_sdpa_repair(model, base, ids + 13, intervals)
    actual, _ = packed_interval_repair(shim, base, ids + 13, intervals)
    assert_ownership_and_untouched(actual, base, snap, intervals)
    for i in range(2):
        for c in (0, 1):
            assert_within_native_precision_floor(ref.layer_kv(actual, i)[c].index_select(2, positions),
                                                 ref.layer_kv(native, i)[c].index_select(2, positions),
                                                 ref.layer_kv(control, i)[c].index_select(2, positions))
            assert_north_star_close(ref.layer_kv(actual, i)[c].index_select(2, positions),
                                    ref.layer_kv(native, i)[c].index_select(2, positions),
                                    ref.layer_kv(control, i)[c].index_select(2, positions))
    query = torch.tensor([[77, 78]], device=gpu_device)
    with torch.no_grad():
        got = model(input_ids=query, past_key_values=ref.clone_cache(actual)).logits
        nat = model(input_ids=query, past_key_values=ref.clone_cache(native)).logits
        ctl = control_model(input_ids=query, past_key_values=ref.clone_cache(control)).logits
    assert_within_native_precision_floor(got, nat, ctl)


def test_config1_shift_and_packed_refresh_match_reference(gpu_device):
    """BASELINE config 1 end to end: tiny random Llama (fp32, seed 0), 256 ids,
    delete 64-95, rotate the 160-row suffix by -32, refresh 8 rows in 2
    intervals [(100,104),(180,184)] through all layers."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from kv_cache_repair_amd.cache import OperatorShim, build_halo_cache
    from kv_cache_repair_amd.kernels.packed_cache import packed_refresh_owned_

    torch.manual_seed(0)
    model = LlamaForCausalLM(LlamaConfig(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                         num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                         rope_theta=10000.0, max_position_embeddings=512)).to(gpu_device).eval()
    gen = torch.Generator().manual_seed(0)
    old_ids = torch.randint(0, 512, (1, 256), generator=gen).to(gpu_device)
    new_ids = torch.cat((old_ids[:, :64], old_ids[:, 96:]), dim=1)
    with torch.no_grad():
        old = model(input_ids=old_ids, use_cache=True).past_key_values
    intervals = [(100, 104), (180, 184)]
    shim = OperatorShim(model)
    ours, meta = build_halo_cache(shim, old, old_ids, new_ids, 0)
    receipt = packed_refresh_owned_(shim, ours, new_ids, intervals)
    expect = ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)
    assert meta["suffix"] >= 160 and receipt["recomputed_tokens"] == 8
    for i in range(2):
        for c in (0, 1):
            torch.testing.assert_close(ref.layer_kv(ours, i)[c], ref.layer_kv(expect, i)[c], rtol=1e-5, atol=2e-6)


def test_bf16_8b_layer_geometry_refresh_matches_reference(gpu_device):
    """Two decoder layers at the 8B geometry (hidden 4096, 32/8 heads x 128,
    theta 5e5, bf16) on a 2048-token cache with BASELINE config 2's edit and
    64-row support: HIP stage vs reference stage on the same GPU."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from kv_cache_repair_amd.cache import OperatorShim, build_halo_cache
    from kv_cache_repair_amd.kernels.packed_cache import packed_refresh_owned_

    torch.manual_seed(1)
    cfg = LlamaConfig(vocab_size=1024, hidden_size=4096, intermediate_size=14336, num_hidden_layers=2,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=500000.0,
                      max_position_embeddings=8192)
    with torch.device(gpu_device):
        model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    gen = torch.Generator(device=gpu_device).manual_seed(1)
    old = ref.cache_from_tensors([(torch.randn(1, 8, 2048, 128, device=gpu_device, generator=gen).to(torch.bfloat16),
                                   torch.randn(1, 8, 2048, 128, device=gpu_device, generator=gen).to(torch.bfloat16))
                                  for _ in range(2)])
    old_ids = torch.randint(0, 1024, (1, 2048), device=gpu_device, generator=gen)
    old_ids[0, 512] = (old_ids[0, 640] + 1) % 1024  # keep the shared prefix at exactly 512 tokens
    new_ids = torch.cat((old_ids[:, :512], old_ids[:, 640:]), dim=1)
    intervals = [(928, 992)]
    shim = OperatorShim(model)
    ours, meta = build_halo_cache(shim, old, old_ids, new_ids, 0)
    packed_refresh_owned_(shim, ours, new_ids, intervals)
    expect = ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)
    control_model = copy.deepcopy(model).float()
    control_old = ref.cache_from_tensors([(l.keys.float(), l.values.float()) for l in old.layers])
    control = ref.reference_refresh_stage(control_model, control_old, old_ids, new_ids, intervals)
    assert meta["position_shift"] == -128
    for i in range(2):
        for c in (0, 1):
            a, e = ref.layer_kv(ours, i)[c], ref.layer_kv(expect, i)[c]
            keep = [p for p in range(a.shape[2]) if not 928 <= p < 992]
            assert bits_equal(a[:, :, keep], e[:, :, keep])  # rotated/copied rows: bit-exact
            assert_north_star_close(a[:, :, 928:992], e[:, :, 928:992], ref.layer_kv(control, i)[c][:, :, 928:992])
            assert_within_native_precision_floor(a[:, :, 928:992], e[:, :, 928:992],
                                                 ref.layer_kv(control, i)[c][:, :, 928:992])


def _large_geometry_stage(gpu_device, family, total, delete_at, delete_span, intervals, seed, layers=2):
    """BASELINE c4 / c5 edits on `layers` decoder layers of the 8B geometry (random
    weights, K/V ~ N(0,1)): HIP stage, reference stage and its fp32 control."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    from kv_cache_repair_amd.cache import OperatorShim, build_halo_cache
    from kv_cache_repair_amd.kernels.packed_cache import packed_refresh_owned_

    torch.manual_seed(seed)
    common = dict(vocab_size=1024, hidden_size=4096, num_hidden_layers=layers, num_attention_heads=32,
                  num_key_value_heads=8, head_dim=128, max_position_embeddings=total)
    if family == "qwen3":
        cfg = Qwen3Config(intermediate_size=12288, rope_theta=1000000.0, layer_types=["full_attention"] * layers,
                          **common)
        ctor = Qwen3ForCausalLM
    else:
        cfg = LlamaConfig(intermediate_size=14336, rope_theta=500000.0, **common)
        ctor = LlamaForCausalLM
    with torch.device(gpu_device):
        model = ctor(cfg).to(torch.bfloat16).eval()
    gen = torch.Generator(device=gpu_device).manual_seed(seed)
    old = ref.cache_from_tensors([(torch.randn(1, 8, total, 128, device=gpu_device, generator=gen).to(torch.bfloat16),
                                   torch.randn(1, 8, total, 128, device=gpu_device, generator=gen).to(torch.bfloat16))
                                  for _ in range(layers)])
    old_ids = torch.randint(0, 1024, (1, total), device=gpu_device, generator=gen)
    old_ids[0, delete_at] = (old_ids[0, delete_at + delete_span] + 1) % 1024  # prefix stops at the edit
    new_ids = torch.cat((old_ids[:, :delete_at], old_ids[:, delete_at + delete_span:]), dim=1)
    shim = OperatorShim(model)
    ours, meta = build_halo_cache(shim, old, old_ids, new_ids, 0)
    receipt = packed_refresh_owned_(shim, ours, new_ids, intervals)
    expect = ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)
    control_model = copy.deepcopy(model).float()
    control_old = ref.cache_from_tensors([(l.keys.float(), l.values.float()) for l in old.layers])
    control = ref.reference_refresh_stage(control_model, control_old, old_ids, new_ids, intervals)
    assert meta["position_shift"] == -delete_span
    assert receipt["recomputed_tokens"] == sum(e - b for b, e in intervals)
    selected = [p for b, e in intervals for p in range(b, e)]
    keep = torch.ones(new_ids.shape[1], dtype=torch.bool, device=gpu_device)
    keep[selected] = False
    for i in range(layers):
        for c in (0, 1):
            a, e = ref.layer_kv(ours, i)[c], ref.layer_kv(expect, i)[c]
            assert bits_equal(a[:, :, keep], e[:, :, keep])  # rotated/copied rows: bit-exact
            assert_north_star_close(a[:, :, selected], e[:, :, selected], ref.layer_kv(control, i)[c][:, :, selected])
            assert_within_native_precision_floor(a[:, :, selected], e[:, :, selected],
                                                 ref.layer_kv(control, i)[c][:, :, selected])


def test_c4_qwen3_geometry_32k_cache_5_percent_budget(gpu_device):
    """BASELINE config 4 on two layers: Qwen3-8B geometry (per-head q/k norm,
    theta 1e6), 32768-token cache, delete 1024 @4096, 1383 rows in 32 random
    intervals (seed 3) -- more rows than one projection launch, so the layers
    run through the dispatched fused shells and the modules' GEMMs."""
    import random

    slots = sorted(random.Random(3).sample(range(27648 // 88), 32))
    intervals = [(4096 + 88 * s, 4096 + 88 * s + (44 if i < 7 else 43)) for i, s in enumerate(slots)]
    _large_geometry_stage(gpu_device, "qwen3", 32768, 4096, 1024, intervals, seed=3)


def test_c5_full_refresh_geometry(gpu_device):
    """BASELINE config 5 on two layers: 8B Llama geometry, 16384-token cache,
    delete 256 @1024, every one of the 15104 suffix rows refreshed (the packed
    attention becomes a dense causal prefill tile; the scatter rewrites the
    whole suffix)."""
    _large_geometry_stage(gpu_device, "llama", 16384, 1024, 256, [(1024, 16128)], seed=4)


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_fresh_row_epilogue_is_bit_identical_to_native_rope_and_scatter(gpu_device, family, dtype):
    """The fused epilogue (kvr_rope_scatter_kv inside the attention shells) and the
    plugin path (native apply_rotary_pos_emb, then the cache layer's scatter and
    the registered attention) produce the same cache bits and next-token logits."""
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, family, kv_heads=2, head_dim=64, dtype=dtype, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    fused, _ = packed_interval_repair(shim, base, edited, intervals, fused_layers=False, fused_projections=False)
    plain, _ = packed_interval_repair(shim, base, edited, intervals, fused_epilogue=False, fused_layers=False,
                                      fused_projections=False)
    for a, b in zip(fused.layers, plain.layers):
        assert bits_equal(a.keys, b.keys) and bits_equal(a.values, b.values)
    with torch.no_grad():
        nxt = torch.tensor([[5]], device=gpu_device)
        la = model(input_ids=nxt, past_key_values=fused, use_cache=True).logits
        lb = model(input_ids=nxt, past_key_values=plain, use_cache=True).logits
    assert bits_equal(la, lb)


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_layers_match_native_layer_ops(gpu_device, family, dtype):
    """Fused RMSNorm / residual / SiLU-gate launches vs the native eager layer ops:
    fp32 within rtol 1e-5 / atol 1e-5 (the reference's packed-vs-sequential
    bound, tests/test_packed_cache.py:74-99, with atol widened from 2e-6: the
    norms' summation order differs; fp32 requests default to the eager ops and
    keep the 2e-6 bound in the other tests); bf16 caches: >= 99% of elements within
    two bf16 ulps of the native path's value (one-ulp norm differences carry
    through later layers) and per-row cosine >= 0.9999."""
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, family, kv_heads=2, head_dim=64, dtype=dtype, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    fused, _ = packed_interval_repair(shim, base, edited, intervals, fused_layers=True, fused_projections=False)
    plain, _ = packed_interval_repair(shim, base, edited, intervals, fused_layers=False, fused_projections=False)
    for a, b in zip(fused.layers, plain.layers):
        for x, y in ((a.keys, b.keys), (a.values, b.values)):
            if dtype == torch.float32:
                torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-5)
            else:
                xf, yf = x.float(), y.float()
                ulp = torch.clamp(yf.abs(), min=2.0 ** -20) * 2.0 ** -7
                assert ((xf - yf).abs() <= 2 * ulp).float().mean().item() >= 0.99
                cos = torch.nn.functional.cosine_similarity(xf.reshape(-1, 64), yf.reshape(-1, 64), dim=-1)
                assert cos.min().item() >= 0.9999


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_projection_plans_match_module_linears(gpu_device, family, dtype):
    """kvr_linear_multi projections (q/k/v in one launch; separate for fp16 Qwen3,
    whose per-head norms then run on their own; gate/up with the SiLU gate in one) vs the modules'
    library GEMMs: both round fp32 accumulations once, so the refreshed caches
    agree to the bf16/fp16 floor: >= 99% of elements within two ulps, per-row
    cosine >= 0.9999. The plans are cached per layer and follow weight moves."""
    from kv_cache_repair_amd.kernels import packed_cache as pc

    model = make_model(gpu_device, family, kv_heads=2, head_dim=64, dtype=dtype, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    fused, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=True)
    plain, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=False)
    eps = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    for a, b in zip(fused.layers, plain.layers):
        for x, y in ((a.keys, b.keys), (a.values, b.values)):
            xf, yf = x.float(), y.float()
            ulp = torch.clamp(yf.abs(), min=2.0 ** -20) * eps
            assert ((xf - yf).abs() <= 2 * ulp).float().mean().item() >= 0.99
            cos = torch.nn.functional.cosine_similarity(xf.reshape(-1, 64), yf.reshape(-1, 64), dim=-1)
            assert cos.min().item() >= 0.9999
    decoder = shim._base_transformer(model)
    plans = [pc._layer_plans(layer) for layer in decoder.layers]
    assert all(p is not None for p in plans)
    # q/k/v in one launch, except fp16 Qwen3 (its per-head norms run as separate launches)
    assert all((p.qkv is None) == (family == "qwen3" and dtype == torch.float16) for p in plans)
    assert pc._layer_plans(decoder.layers[0]) is plans[0]  # cached
    again, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=True)
    assert all(torch.equal(x.keys, y.keys) and torch.equal(x.values, y.values)
               for x, y in zip(again.layers, fused.layers))  # deterministic
    with torch.no_grad():  # a weight moved to new storage invalidates that layer's plans
        layer0 = decoder.layers[0]
        layer0.mlp.down_proj.weight.data = layer0.mlp.down_proj.weight.data.clone()
    assert pc._layer_plans(layer0) is not plans[0]
    moved, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=True)
    assert all(torch.equal(x.keys, y.keys) for x, y in zip(moved.layers, fused.layers))



@pytest.mark.parametrize("head_dim", [96, 8])
def test_bf16_qwen3_head_dims_outside_the_vector_epilogue(gpu_device, head_dim):
    """bf16 Qwen3 with a head dim whose half row is not a power-of-two count of
    16-byte chunks (96: 6 chunks; 8: 8 bytes): the fresh-row epilogue's vector
    kernel cannot fold the per-head q/k norms in, so both the Python-dispatched
    shells and kvr_decoder_layer run them as kvr_rms_norm launches before the
    plain epilogue. The refresh runs by default, native and dispatched layers are
    bit-identical, and the cache agrees with the module path (hipBLASLt GEMMs,
    eager norms and RoPE) to the bf16 floor."""
    from kv_cache_repair_amd.kernels import packed_cache as pc

    model = make_model(gpu_device, "qwen3", kv_heads=2, head_dim=head_dim, dtype=torch.bfloat16, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    snap = snapshot(base)
    default, receipt = pc.packed_interval_repair(shim, base, edited, intervals)
    native, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)
    dispatched, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=False)
    plain, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_epilogue=False, fused_layers=False,
                                         fused_projections=False)
    assert_ownership_and_untouched(default, base, snap, intervals)
    decoder = shim._base_transformer(model)
    assert all(pc._layer_plans(layer).qkv is None for layer in decoder.layers)  # q, k, v launched apart
    n = edited.shape[1]
    for a, b, c, d in zip(default.layers, native.layers, dispatched.layers, plain.layers):
        for w, x, y, z in ((a.keys, b.keys, c.keys, d.keys), (a.values, b.values, c.values, d.values)):
            assert bits_equal(w, x) and bits_equal(x, y)
            xf, zf = x.float(), z.float()
            ulp = torch.clamp(zf.abs(), min=2.0 ** -20) * 2.0 ** -7
            assert ((xf - zf).abs() <= 2 * ulp).float().mean().item() >= 0.99
            rows_x = xf.permute(0, 2, 1, 3).reshape(n, -1)
            rows_z = zf.permute(0, 2, 1, 3).reshape(n, -1)
            assert torch.nn.functional.cosine_similarity(rows_x, rows_z, dim=-1).min().item() >= 0.9999


def test_model_changes_between_refreshes_are_seen(gpu_device):
    """The executor caches the model's qualification and layer plans under a
    fingerprint of the module tree (module and parameter identities, storage
    addresses). Between two refreshes: new weight values in new storage are
    used (not the cached pointers), a replaced module is seen, and a
    parameter moved off the GPU is refused as on a first call."""
    from kv_cache_repair_amd.kernels import packed_cache as pc

    dtype = torch.bfloat16
    model = make_model(gpu_device, "llama", kv_heads=2, head_dim=64, dtype=dtype, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    decoder = shim._base_transformer(model)

    def close_to_module_linears(native):
        plain, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=False)
        for a, b in zip(native.layers, plain.layers):
            for x, y in ((a.keys, b.keys), (a.values, b.values)):
                xf, yf = x.float(), y.float()
                ulp = torch.clamp(yf.abs(), min=2.0 ** -20) * 2.0 ** -7
                assert ((xf - yf).abs() <= 2 * ulp).float().mean().item() >= 0.99
                cos = torch.nn.functional.cosine_similarity(xf.reshape(-1, 64), yf.reshape(-1, 64), dim=-1)
                assert cos.min().item() >= 0.9999

    first, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)
    close_to_module_linears(first)
    with torch.no_grad():  # new values in new storage; the old storage is released
        proj = decoder.layers[0].self_attn.v_proj
        proj.weight.data = (proj.weight.data.float() * -1.5).to(dtype)
    changed, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)
    assert not torch.equal(changed.layers[2].values, first.layers[2].values)
    close_to_module_linears(changed)
    with torch.no_grad():  # a replaced module holding the same weight tensor, now with a bias
        old = decoder.layers[1].mlp.down_proj
        new = torch.nn.Linear(old.in_features, old.out_features, bias=True, device=gpu_device, dtype=dtype).eval()
        new.weight = old.weight
        new.bias.fill_(0.25)
        decoder.layers[1].mlp.down_proj = new
    replaced, _ = pc.packed_interval_repair(shim, base, edited, intervals)  # plans refused: module path
    assert not torch.equal(replaced.layers[2].keys, changed.layers[2].keys)
    close_to_module_linears(replaced)
    with pytest.raises(ValueError, match="native_layers"):
        pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)
    with torch.no_grad():
        decoder.layers[2].mlp.up_proj.weight.data = decoder.layers[2].mlp.up_proj.weight.data.cpu()
    with pytest.raises(ValueError, match="request device"):
        pc.packed_interval_repair(shim, base, edited, intervals)


def test_forward_hooks_take_the_module_path(gpu_device):
    """A forward hook on a decoder module runs as in the reference's packed
    forward (the modules' own forwards): the fused projections, norms and
    native layers, which would skip it, are off by default and refused when
    asked for; without hooks the fused path is back."""
    from kv_cache_repair_amd.kernels import packed_cache as pc

    model = make_model(gpu_device, "llama", kv_heads=2, head_dim=64, dtype=torch.bfloat16, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    decoder = shim._base_transformer(model)
    calls = []
    handle = decoder.layers[1].self_attn.q_proj.register_forward_hook(lambda m, args, out: calls.append(out.shape))
    try:
        hooked, _ = pc.packed_interval_repair(shim, base, edited, intervals)
        assert calls == [torch.Size([1, 31, 256])]  # the hooked projection ran once, over the 31 selected rows
        plain, _ = pc.packed_interval_repair(shim, base, edited, intervals, fused_projections=False,
                                             fused_layers=False, native_layers=False)
        assert all(torch.equal(a.keys.view(torch.int16), b.keys.view(torch.int16))
                   and torch.equal(a.values.view(torch.int16), b.values.view(torch.int16))
                   for a, b in zip(hooked.layers, plain.layers))
        for option in ("native_layers", "fused_projections", "fused_layers"):
            with pytest.raises(ValueError, match="module path"):
                pc.packed_interval_repair(shim, base, edited, intervals, **{option: True})
    finally:
        handle.remove()
    calls.clear()
    pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)  # accepted again
    assert calls == []


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_native_layer_call_is_bit_identical_to_dispatched_fused_layers(gpu_device, family, dtype):
    """kvr_decoder_layer enqueues the same kernels with the same arguments as the
    Python-dispatched fused shells, so the refreshed caches are bit-identical;
    it is the default whenever the fusions are active, and refuses requests
    it cannot serve instead of falling back silently."""
    from kv_cache_repair_amd.kernels import packed_cache as pc

    model = make_model(gpu_device, family, kv_heads=2, head_dim=64, dtype=dtype, layers=3)
    shim, ids, base = make_request(model, length=140)
    edited = ids.clone()
    edited[0, 70:] = (edited[0, 70:] + 7) % 97
    intervals = [(0, 2), (5, 9), (63, 70), (100, 117), (139, 140)]
    native, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True)
    dispatched, _ = pc.packed_interval_repair(shim, base, edited, intervals, native_layers=False)
    default, _ = pc.packed_interval_repair(shim, base, edited, intervals)
    for a, b, c in zip(native.layers, dispatched.layers, default.layers):
        for x, y, z in ((a.keys, b.keys, c.keys), (a.values, b.values, c.values)):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))
            assert torch.equal(x.view(torch.int16), z.view(torch.int16))
    with pytest.raises(ValueError, match="native_layers"):
        pc.packed_interval_repair(shim, base, edited, intervals, native_layers=True, fused_projections=False)
    with pytest.raises(ValueError, match="native_layers"):  # more rows than one projection launch serves
        pc.packed_interval_repair(shim, base, edited, [(0, 65)], native_layers=True)


def test_cache_layer_off_the_request_device_is_refused(gpu_device):
    """One layer's K and V on the host: the one-pass layout read sees two devices
    and the per-layer device check names the problem before any launch."""
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    model = make_model(gpu_device, layers=3)
    shim, ids, base = make_request(model)
    base.layers[1].keys, base.layers[1].values = base.layers[1].keys.cpu(), base.layers[1].values.cpu()
    with pytest.raises(ValueError, match="cache layers on the request device"):
        packed_interval_repair(shim, base, ids + 13, [(3, 5), (8, 10)])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_owned_refresh_with_one_layer_at_other_strides_matches_uniform_layout(gpu_device, dtype):
    """A cache whose layers do not share one layout takes the per-tensor reads
    (validation, device check, per-layer descriptors): same bits as the same
    values in one uniform layout."""
    from kv_cache_repair_amd.kernels.packed_cache import packed_refresh_owned_

    model = make_model(gpu_device, layers=3, dtype=dtype)
    shim, ids, base = make_request(model)
    uniform, mixed = ref.clone_cache(base), ref.clone_cache(base)
    layer = mixed.layers[1]
    layer.keys = layer.keys.transpose(1, 2).contiguous().transpose(1, 2)  # token-major storage, same values
    layer.values = layer.values.transpose(1, 2).contiguous().transpose(1, 2)
    assert layer.keys.stride() != uniform.layers[1].keys.stride()
    intervals = [(0, 1), (3, 5), (8, 10)]
    packed_refresh_owned_(shim, uniform, ids + 13, intervals)
    packed_refresh_owned_(shim, mixed, ids + 13, intervals)
    for a, b in zip(uniform.layers, mixed.layers):
        assert bits_equal(a.keys, b.keys) and bits_equal(a.values, b.values)
