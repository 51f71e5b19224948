#!/usr/bin/env python3
"""Refresh-stage benchmark of the MI355X packed refresh executor (one GPU).

Headline workload (the metric's config, the default):
an 8B-shaped Llama (32 layers, hidden 4096, MLP 14336, 32 query / 8 KV heads x
128, RoPE theta 5e5, vocab 128256, random init, bf16); a synthetic 8192-token
cache with K/V ~ N(0,1) (seed 1); a 512-token deletion at position 2048 (shift
-512, 5632-row suffix); a 64-token budget as 16 intervals of 4 rows at random
suffix slots (seed 2).

One step = one full refresh stage, inputs resident in HBM: shift-cache build
(prefix copy + RoPE delta rotation of every suffix K row + V copy, all layers)
-> plan upload -> packed forward through all layers with, per layer, the
projections, the norms, the fused fresh-row epilogue (RoPE of the fresh Q/K +
K/V scatter) and the packed attention. Prefill, tokenisation and selection are
outside the step, as in the reference benchmark (benchmark_refresh.py:3-9);
unlike it, the rotation is inside. The build reads the token ids from host
copies, as repair_after_deletion does (its tokenizer output is on the host), so
the step issues no device-to-host copy; the reference path keeps its own
device-id read (cache.py:116-117).

Printed (one JSON line): stage latency in ms per repair (value = the median of
the K steps' per-call samples, each call bracketed by torch.cuda.synchronize()
as the reference benchmark times it, benchmark_refresh.py:106-126; with p95 and
the back-to-back figure beside it), the same stage run the reference way on the
same GPU, the device time of every
libkvrepair kernel of the step (HIP events around replays of a graph of
back-to-back launches of that kernel with the stage's own shapes: no host time
inside), a roofline object for the dominant kernel and one per north-star
kernel (rotate, shift-cache build, scatter, fresh-row epilogue, attention),
the end-to-end parity checks at full depth against the reference path and an
fp32 control plus the teacher-forced per-layer north-star check, the selection
scorer, and the reference stage timed on the host CPU over all layers
(cpu_baseline).

Other modes (secondary lines, not the headline):
  --workload c2|c4|c5   the same measurements on BASELINE configs 2, 4, 5 at
                        full depth, with kernel-level CPU timings;
  --grid                the reference benchmark's grid (lengths 2048/8192 x
                        1/4/16 intervals, 64-token budget, refresh only:
                        benchmark_refresh.py:35-49, 129-182), one line per case.
"""

from __future__ import annotations

import argparse
import contextlib
import copy
import ctypes
import gc
import json
import math
import os
import random
import statistics
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "budgeted-kv-cache-repair_amd"), str(ROOT)]

import torch  # noqa: E402

METRIC = "refresh-stage latency (ms) per repair at 8k ctx/64-tok budget; rotate GB/s"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


# ----------------------------------------------------------------------------- workloads
@dataclass(frozen=True)
class Workload:
    """One BASELINE configuration: model geometry, cache, edit and support."""

    name: str
    family: str  # "llama" or "qwen3"
    layers: int
    hidden: int
    mlp: int
    hq: int
    hkv: int
    dim: int
    vocab: int
    theta: float
    total: int         # prefilled (old) cache length
    delete_at: int
    delete_span: int
    seed: int          # weights and K/V
    description: str
    support: tuple = field(default=())

    @property
    def edited(self) -> int:
        return self.total - self.delete_span

    @property
    def suffix(self) -> int:
        return self.total - self.delete_at - self.delete_span

    def intervals(self) -> list[tuple[int, int]]:
        return [tuple(iv) for iv in self.support]

    def positions(self) -> list[int]:
        return [p for s, e in self.intervals() for p in range(s, e)]


def c3_intervals() -> list[tuple[int, int]]:
    """16 intervals of 4 rows at random 8-token slots of the c3 suffix (seed 2)."""
    suffix = 8192 - 2048 - 512
    slots = sorted(random.Random(2).sample(range(suffix // 8), 16))
    return [(2048 + 8 * s, 2048 + 8 * s + 4) for s in slots]


def c4_intervals() -> list[tuple[int, int]]:
    """ceil(5% of 27648) = 1383 rows: 7 intervals of 44 and 25 of 43 at random
    88-token slots of the c4 suffix (seed 3)."""
    slots = sorted(random.Random(3).sample(range(27648 // 88), 32))
    return [(4096 + 88 * s, 4096 + 88 * s + (44 if i < 7 else 43)) for i, s in enumerate(slots)]


_LLAMA8B = dict(family="llama", layers=32, hidden=4096, mlp=14336, hq=32, hkv=8, dim=128, vocab=128256,
                theta=500000.0)
WORKLOADS = {
    "c2": Workload("c2", total=2048, delete_at=512, delete_span=128, seed=1, support=((928, 992),),
                   description="c2: 8B-shaped Llama, 2048-token cache, delete 128 @512, 64 rows in 1 interval",
                   **_LLAMA8B),
    "c3": Workload("c3", total=8192, delete_at=2048, delete_span=512, seed=1, support=tuple(c3_intervals()),
                   description="c3: 8B-shaped Llama, 8192-token cache, delete 512 @2048, 64-token budget in 16x4",
                   **_LLAMA8B),
    "c4": Workload("c4", family="qwen3", layers=36, hidden=4096, mlp=12288, hq=32, hkv=8, dim=128, vocab=151936,
                   theta=1000000.0, total=32768, delete_at=4096, delete_span=1024, seed=3,
                   support=tuple(c4_intervals()),
                   description="c4: Qwen3-8B-shaped, 32768-token cache, delete 1024 @4096, 5% budget (1383 rows) "
                               "in 32 intervals"),
    "c5": Workload("c5", total=16384, delete_at=1024, delete_span=256, seed=4, support=((1024, 16128),),
                   description="c5: 8B-shaped Llama, 16384-token cache, delete 256 @1024, 100% budget "
                               "(15104 rows)", **_LLAMA8B),
}
C3 = WORKLOADS["c3"]

# headline (c3) geometry, kept as module constants for callers
LAYERS, HIDDEN, MLP, HQ, HKV, DIM, VOCAB, THETA = C3.layers, C3.hidden, C3.mlp, C3.hq, C3.hkv, C3.dim, C3.vocab, \
    C3.theta
TOTAL, DELETE_AT, DELETE_SPAN, BUDGET_INTERVALS, ROWS_PER_INTERVAL = C3.total, C3.delete_at, C3.delete_span, 16, 4


def make_model(device, workload: Workload = C3, layers: int | None = None, seed: int | None = None,
               dtype=torch.bfloat16, vocab: int | None = None):
    """Random-init model of the workload's shape on ``device``.

    Built on the meta device and materialised directly: linear and embedding
    weights ~ N(0, 0.02) (drawn in fp32, cast to ``dtype``), RMSNorm weights
    (q/k norms included) 1, RoPE buffers recomputed -- the values HF's own init
    gives, without its slow per-element sampling on the host.
    """
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    w = workload
    n_layers = w.layers if layers is None else layers
    common = dict(vocab_size=w.vocab if vocab is None else vocab, hidden_size=w.hidden, intermediate_size=w.mlp,
                  num_hidden_layers=n_layers, num_attention_heads=w.hq, num_key_value_heads=w.hkv, head_dim=w.dim,
                  rope_theta=w.theta, max_position_embeddings=w.total)
    if w.family == "qwen3":
        cfg, ctor = Qwen3Config(layer_types=["full_attention"] * n_layers, **common), Qwen3ForCausalLM
    else:
        cfg, ctor = LlamaConfig(**common), LlamaForCausalLM
    previous = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device("meta"):
            model = ctor(cfg)
    finally:
        torch.set_default_dtype(previous)
    model = model.to_empty(device=device).eval()
    gen = torch.Generator(device=device).manual_seed(w.seed if seed is None else seed)
    with torch.no_grad():
        for name, param in model.named_parameters():
            if name.endswith("norm.weight"):
                param.fill_(1.0)
                continue
            flat = param.view(-1)
            for start in range(0, flat.numel(), 1 << 26):
                chunk = flat[start:start + (1 << 26)]
                chunk.copy_(torch.empty(chunk.numel(), device=device).normal_(0.0, 0.02, generator=gen))
        rotary = model.model.rotary_emb
        inv_freq, scaling = rotary.compute_default_rope_parameters(cfg, device)
        rotary.inv_freq = inv_freq.to(device=device, dtype=torch.float32)
        rotary.original_inv_freq = rotary.inv_freq.clone()
        rotary.attention_scaling = scaling
    model.set_attn_implementation("sdpa")
    return model


def make_request(device, workload: Workload = C3, layers: int | None = None, vocab: int | None = None):
    """Synthetic stale cache (K/V ~ N(0,1), bf16, workload seed) and the workload's edit:
    old ids random, the shared prefix kept exactly ``delete_at`` tokens long."""
    from kv_cache_repair_amd.cache import cache_from_tensors

    w = workload
    n_layers = w.layers if layers is None else layers
    n_vocab = w.vocab if vocab is None else vocab
    gen = torch.Generator(device=device).manual_seed(w.seed)
    pairs = [(torch.randn(1, w.hkv, w.total, w.dim, device=device, generator=gen, dtype=torch.bfloat16),
              torch.randn(1, w.hkv, w.total, w.dim, device=device, generator=gen, dtype=torch.bfloat16))
             for _ in range(n_layers)]
    old_ids = torch.randint(0, n_vocab, (1, w.total), device=device, generator=gen)
    old_ids[0, w.delete_at] = (old_ids[0, w.delete_at + w.delete_span] + 1) % n_vocab
    new_ids = torch.cat((old_ids[:, :w.delete_at], old_ids[:, w.delete_at + w.delete_span:]), dim=1)
    return cache_from_tensors(pairs), old_ids, new_ids


# ----------------------------------------------------------------------------- our stage
def hip_stage(shim, old, old_ids, new_ids, intervals, native_layers=None, host_ids=None):
    """The refresh stage as repair_after_deletion runs it after selection: the
    shift-cache build, then the packed refresh in place. ``host_ids`` (the old and
    edited ids on the host, as the API layer holds them from its tokenizer) let
    the build read the ids without a device synchronisation."""
    from kv_cache_repair_amd.cache import build_halo_cache
    from kv_cache_repair_amd.kernels.packed_cache import packed_refresh_owned_

    build_old, build_new = host_ids if host_ids is not None else (old_ids, new_ids)
    cache, _ = build_halo_cache(shim, old, build_old, build_new, 0)
    packed_refresh_owned_(shim, cache, new_ids, intervals, native_layers=native_layers)
    return cache


@contextlib.contextmanager
def no_gc():
    """Python's cyclic garbage collector paused (timed regions of both paths:
    a collection pass during a few hundred launches is a host stall of tens
    of ms)."""
    enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if enabled:
            gc.enable()


def time_calls(fn, steps, warmup) -> dict:
    """The reference benchmark's timing (benchmark_refresh.py:106-126): ``warmup``
    untimed calls, then ``steps`` calls each bracketed by torch.cuda.synchronize()
    on both sides, so every sample is one whole repair from host entry to device
    completion. Returns the median, p95, mean and raw samples (ms)."""
    for _ in range(warmup):
        out = fn()
        torch.cuda.synchronize()
        del out
    samples = []
    with no_gc():
        torch.cuda.synchronize()
        for _ in range(steps):
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            samples.append((time.perf_counter() - t0) * 1000.0)
            del out
    ordered = sorted(samples)
    return {"median_ms": statistics.median(samples), "p95_ms": ordered[min(len(ordered) - 1,
                                                                             math.ceil(0.95 * len(ordered)) - 1)],
            "mean_ms": statistics.fmean(samples), "min_ms": ordered[0], "samples_ms": samples}


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        out = fn()
        torch.cuda.synchronize()
        del out
    with no_gc():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = fn()
            del out
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    return elapsed * 1000.0 / steps


# ----------------------------------------------------------------------------- reference stage (same GPU)
@torch.no_grad()
def reference_stage(model, old, old_ids, new_ids, intervals, shifted=None, record=None):
    """The reference's eager path on this GPU: build_halo_cache with the per-layer
    rotate chain and cats (cache.py:103-144), clone_cache, boolean mask and
    index_copy_ + HF sdpa_attention_forward per layer (packed_cache.py:179-298).
    With ``shifted`` (a shifted cache) only the packed refresh runs, as the
    reference benchmark times it (benchmark_refresh.py:129-164). ``record``
    (a dict) receives the shifted cache (``shifted``) and, per decoder layer,
    its input hidden rows (``inputs[i]``) and attention output (``attention[i]``,
    [1, B, Hq, D]), plus the selected rows' rotary tables (``tables``)."""
    from transformers.cache_utils import Cache, DynamicLayer
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    from kv_cache_repair_amd.cache import cache_from_tensors

    base = model.model
    name = "bench_reference_packed_sdpa"
    if name not in ALL_ATTENTION_FUNCTIONS:
        def attend(module, q, k, v, mask, *, scaling=None, dropout=0.0, bench_mask=None, bench_record=None, **kw):
            out, weights = sdpa_attention_forward(module, q, k, v, bench_mask, dropout=0.0, scaling=scaling,
                                                  is_causal=False)
            if bench_record is not None:
                bench_record["attention"][module.layer_idx] = out.detach().clone()
            return out, weights
        ALL_ATTENTION_FUNCTIONS.register(name, attend)

    if shifted is None:
        # build_halo_cache: host alignment, prefix clone, rotate chain, cats
        old_l = [int(x) for x in old_ids[0].tolist()]
        new_l = [int(x) for x in new_ids[0].tolist()]
        prefix = 0
        while prefix < min(len(old_l), len(new_l)) and old_l[prefix] == new_l[prefix]:
            prefix += 1
        suffix = 0
        while suffix < min(len(old_l), len(new_l)) - prefix and old_l[-1 - suffix] == new_l[-1 - suffix]:
            suffix += 1
        shift = (len(new_l) - suffix) - (len(old_l) - suffix)
        ots = len(old_l) - suffix
        pairs = []
        for layer in old.layers:
            k, v = layer.keys, layer.values
            pk, pv = k[:, :, :prefix].clone(), v[:, :, :prefix].clone()
            tail = k[:, :, ots:]
            pos = torch.full((1, tail.shape[2]), shift, dtype=torch.long, device=tail.device)
            cos, sin = base.rotary_emb(tail, pos)
            cos, sin = cos.unsqueeze(1).to(tail.dtype), sin.unsqueeze(1).to(tail.dtype)
            half = tail.shape[-1] // 2
            rot = torch.cat((-tail[..., half:], tail[..., :half]), dim=-1)
            nk = torch.cat((pk, tail * cos + rot * sin), dim=2)
            nv = torch.cat((pv, v[:, :, ots:].clone()), dim=2)
            pairs.append((torch.cat((torch.empty_like(nk[:, :, :0]), nk), dim=2),
                          torch.cat((torch.empty_like(nv[:, :, :0]), nv), dim=2)))  # DynamicLayer.update cat
    else:
        pairs = [(layer.keys, layer.values) for layer in shifted.layers]
    if record is not None:
        record.update(shifted=cache_from_tensors(pairs), inputs={}, attention={}, tables=None)
    # packed_interval_repair (sdpa + torch writeback)
    selected = [p for s, e in intervals for p in range(s, e)]
    positions = torch.tensor(selected, dtype=torch.long, device=new_ids.device)
    length = new_ids.shape[1]
    mask = (torch.arange(length, device=new_ids.device)[None, :] <= positions[:, None])[None, None]
    output = cache_from_tensors([(k.clone(), v.clone()) for k, v in pairs])

    class _Layer(DynamicLayer):
        def __init__(self, k, v):
            super().__init__()
            self.keys, self.values, self.is_initialized = k, v, True
            self.dtype, self.device = k.dtype, k.device

        def update(self, ks, vs, *a, **kw):
            self.keys.index_copy_(2, positions, ks)
            self.values.index_copy_(2, positions, vs)
            return self.keys, self.values

        def get_mask_sizes(self, query_length):
            return length, 0

    config = copy.deepcopy(base.config)
    config._attn_implementation = name
    view = copy.copy(base)
    view._modules = base._modules.copy()
    view.config = config
    layers = []
    for original in base.layers:
        layer = copy.copy(original)
        layer._modules = original._modules.copy()
        attn = copy.copy(original.self_attn)
        attn._modules = original.self_attn._modules.copy()
        attn.config = config
        layer._modules["self_attn"] = attn
        if record is not None:
            layer.forward = _recording_forward(layer.forward, len(layers), record)
        layers.append(layer)
    view._modules["layers"] = torch.nn.ModuleList(layers)
    cache = Cache(layers=[_Layer(l.keys, l.values) for l in output.layers])
    extra = {"bench_record": record} if record is not None else {}
    view(input_ids=new_ids.index_select(1, positions), position_ids=positions[None], past_key_values=cache,
         use_cache=True, bench_mask=mask, **extra)
    return output


def _recording_forward(forward, index, record):
    """A decoder layer's forward that first records its input hidden rows (and,
    at layer 0, the rotary tables of the selected rows)."""
    def run(hidden_states, *args, **kwargs):
        record["inputs"][index] = hidden_states.detach().clone()
        if index == 0:
            record["tables"] = tuple(t.detach().clone() for t in kwargs["position_embeddings"])
        return forward(hidden_states, *args, **kwargs)
    return run


# ----------------------------------------------------------------------------- end-to-end parity at full depth
def sdpa_backend_used(fn) -> dict:
    """Run ``fn`` once (untimed) and record which fused backend torch picks for
    the first ``scaled_dot_product_attention`` call it makes, with that call's
    own arguments (the reference path's boolean mask and repeat_kv'd K/V)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend

    seen = {}
    original = F.scaled_dot_product_attention

    def spy(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, **kwargs):
        if not seen:
            try:
                choice = torch._fused_sdp_choice(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                                                 is_causal=is_causal, scale=scale, **kwargs)
                seen["backend"] = SDPBackend(choice).name
            except Exception as exc:  # private API: record that it could not be asked
                seen["backend"] = f"unknown ({type(exc).__name__})"
            seen["query"] = list(query.shape)
            seen["key"] = list(key.shape)
            seen["mask"] = None if attn_mask is None else f"{attn_mask.dtype} {list(attn_mask.shape)}"
        return original(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal,
                        scale=scale, **kwargs)

    F.scaled_dot_product_attention = spy
    try:
        out = fn()
        torch.cuda.synchronize()
        del out
    finally:
        F.scaled_dot_product_attention = original
    return seen


def row_errors(a: torch.Tensor, b: torch.Tensor) -> dict:
    """max-abs, RMSE and the smallest per-row cosine of a against b (rows = head_dim vectors)."""
    a, b = a.double(), b.double()
    d = a - b
    cos = torch.nn.functional.cosine_similarity(a.reshape(-1, a.shape[-1]), b.reshape(-1, b.shape[-1]), dim=-1)
    return {"max_abs": d.abs().max().item(), "rmse": d.square().mean().sqrt().item(), "min_cos": cos.min().item()}


def depth_parity(ours, theirs, control, positions) -> dict:
    """Per layer and per K/V: the refreshed rows of our cache and of the
    reference path's cache against an fp32 control (the reference's own gate,
    tests/test_packed_cache.py:291-315: ours <= 2 x the reference's error on
    max-abs and RMSE, fp32-eps floor) and against each other; the other rows
    must be bit-identical to the reference's."""
    device = ours.layers[0].keys.device
    n = ours.layers[0].keys.shape[2]
    keep = torch.ones(n, dtype=torch.bool, device=device)
    keep[positions] = False
    index = torch.tensor(positions, dtype=torch.long, device=device)
    rows, bit_exact = [], True
    for i, (o, t, c) in enumerate(zip(ours.layers, theirs.layers, control.layers)):
        for part, a, b, f in (("k", o.keys, t.keys, c.keys), ("v", o.values, t.values, c.values)):
            bit_exact &= bool(torch.equal(a[:, :, keep].view(torch.int16), b[:, :, keep].view(torch.int16)))
            sa, sb, sf = a.index_select(2, index), b.index_select(2, index), f.index_select(2, index)
            floor = torch.finfo(torch.float32).eps * max(1.0, sf.abs().max().item())
            ours_f, ref_f, ours_ref = row_errors(sa, sf), row_errors(sb, sf), row_errors(sa, sb)
            gate = all(ours_f[m] <= 2.0 * max(ref_f[m], floor) for m in ("max_abs", "rmse"))
            rows.append({"layer": i, "part": part, "ours_vs_fp32": ours_f, "reference_vs_fp32": ref_f,
                         "ours_vs_reference": ours_ref, "gate": gate})
    worst = lambda key, m, f: f(r[key][m] for r in rows)  # noqa: E731
    return {
        "unselected_rows_bit_exact_vs_reference": bit_exact,
        "precision_floor_gate_all_layers": all(r["gate"] for r in rows),
        "ours_vs_fp32": {"max_abs": worst("ours_vs_fp32", "max_abs", max), "rmse": worst("ours_vs_fp32", "rmse", max),
                         "min_cos": worst("ours_vs_fp32", "min_cos", min)},
        "reference_vs_fp32": {"max_abs": worst("reference_vs_fp32", "max_abs", max),
                              "rmse": worst("reference_vs_fp32", "rmse", max),
                              "min_cos": worst("reference_vs_fp32", "min_cos", min)},
        "ours_vs_reference": {"max_abs": worst("ours_vs_reference", "max_abs", max),
                              "min_cos": worst("ours_vs_reference", "min_cos", min)},
        "max_error_ratio_vs_reference": max(
            r["ours_vs_fp32"][m] / max(r["reference_vs_fp32"][m], 1e-30) for r in rows for m in ("max_abs", "rmse")),
        "layers": rows,
    }


NORTH_STAR_MAX_ABS = 2e-2
NORTH_STAR_MIN_COS = 0.9999


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """One unit in the last place of bf16 at |x| (2^(e-7) for |x| in [2^e, 2^(e+1)))."""
    _, exponent = torch.frexp(x.float().abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(x, dtype=torch.float32), exponent - 8)


def _north_star(a: torch.Tensor, b: torch.Tensor, rotated: bool = False) -> dict:
    """max-abs, RMSE, smallest per-row cosine (rows = last-dim vectors) of ``a``
    against ``b``, the count of elements beyond 2e-2 and whether each of those
    is within two bf16 ulps of its scale: |b| itself, or for ``rotated`` rows
    (RoPE'd keys) the norm r of the element's rotate-half pair in ``b``.

    Why: a projection rounded once from fp32 by two summation orders can differ
    by one ulp of the projected value, and the normalised input it reads by one
    or two more; RoPE then adds two rounded products k cos and k2 sin, each at
    most r in magnitude (rotation keeps the pair norm), so a rotated key can sit
    two ulps of r away even where it is itself small (cancellation). At r in
    [2, 4) two ulps are 0.031, where 2e-2 is 1.3 ulps."""
    stats = row_errors(a, b)
    bf = b.float()
    d = (a.float() - bf).abs()
    beyond = d > NORTH_STAR_MAX_ABS
    scale = bf.abs()
    if rotated:
        half = bf.shape[-1] // 2
        r = torch.sqrt(bf[..., :half].square() + bf[..., half:].square())
        scale = torch.cat((r, r), dim=-1)
    stats["beyond_2e-2"] = int(beyond.sum().item())
    stats["beyond_2e-2_within_2ulp"] = bool((d[beyond] <= 2 * _bf16_ulp(scale)[beyond]).all().item())
    return stats


@torch.no_grad()
def teacher_forced_parity(model, new_ids, intervals, record, reference_output) -> dict:
    """Each decoder layer of this build fed the reference path's own layer input.

    ``record`` comes from a reference run (bench.reference_stage or the oracle's
    reference_refresh_stage with ``record``): its shifted cache, each layer's
    input hidden rows and attention output, the rotary tables. Layer i of this
    build runs once on ``inputs[i]`` over a copy of that shifted cache with the
    executor's own launches (projection plans, fused RMSNorm, fresh-row
    epilogue, the rounded-probability attention schedule: the Python-dispatched
    shells, which enqueue the same kernels as the native layer call). Its fresh
    K/V rows (scattered into the copy), its attention output and its output
    hidden rows are compared with the reference layer's, so each layer's own
    error is separated from the bf16 drift that accumulates over the depth.
    Where the native layer call serves the model (<= 64 rows), kvr_decoder_layer
    also runs each layer on the same input and must give the same bits.
    """
    import dataclasses

    from transformers.cache_utils import Cache

    from kv_cache_repair_amd import _native
    from kv_cache_repair_amd.cache import cache_from_tensors
    from kv_cache_repair_amd.kernels import packed_cache as pc
    from kv_cache_repair_amd.kernels.indexed_attention import IndexedPlan

    base = model.model
    device = new_ids.device
    n = int(new_ids.shape[1])
    positions = [p for s, e in intervals for p in range(s, e)]
    index = torch.tensor(positions, dtype=torch.long, device=device)
    shifted = record["shifted"]
    n_layers = len(shifted.layers)
    key0 = shifted.layers[0].keys
    plan = IndexedPlan(positions, n).to(device)
    launcher = pc._launcher(plan, base.config, key0)
    plans = pc._projection_plans_for(base, None, key0.dtype, len(positions))
    attended = {}

    def recorder(fn, i):
        def run(x, *args, **kwargs):
            attended[i] = x.detach().clone()
            return fn(x, *args, **kwargs)
        return run

    shell_plans = None
    if plans is not None:
        shell_plans = [dataclasses.replace(p, o=recorder(p.o, i)) for i, p in enumerate(plans)]
    view = pc._make_native_view(base, True, True, shell_plans)
    if plans is None:  # the shells call the o_proj modules: wrap them in the shells only
        for i, layer in enumerate(view.layers):
            shell = layer._modules["self_attn"]
            shell._modules["o_proj"] = recorder(shell._modules["o_proj"], i)
    output = cache_from_tensors([(l.keys.clone(), l.values.clone()) for l in shifted.layers])
    context = pc._PackedContext(plan.positions, n, "hip", plan, launcher)
    cache = Cache(layers=[pc._PackedLayer(l.keys, l.values, context, "hip") for l in output.layers])
    tables = record["tables"]
    hidden_out = {}
    for i, layer in enumerate(view.layers):
        hidden_out[i] = layer(record["inputs"][i].clone(), position_embeddings=tables, past_key_values=cache,
                              use_cache=True, sur_packed_context=context)
    native = None
    if pc._native_layers_for(None, base, plans, True, True):
        native_cache = cache_from_tensors([(l.keys.clone(), l.values.clone()) for l in shifted.layers])
        first = base.layers[0]
        forward = pc._NativeForward(launcher, int(first.mlp.down_proj.weight.shape[0]),
                                    int(first.mlp.gate_proj.weight.shape[0]), float(first.self_attn.scaling))
        forward.bind_tables(tables)
        descs = pc._native_layer_descs(plans, native_cache, n_layers)
        same = True
        for i in range(n_layers):
            desc = descs[i]
            desc.input_normed, desc.next_norm = 0, None  # a single layer: its own input norm, none for the next
            h = record["inputs"][i].clone().contiguous()
            status = _native.lib().kvr_decoder_layer(ctypes.byref(desc), ctypes.byref(forward.desc), h.data_ptr(),
                                                     forward.stream)
            _native.check(status, "kvr_decoder_layer")
            same &= bool(torch.equal(h.view(torch.int16), hidden_out[i].contiguous().view(torch.int16)))
        for a, b in zip(native_cache.layers, output.layers):
            same &= bool(torch.equal(a.keys.view(torch.int16), b.keys.view(torch.int16)))
            same &= bool(torch.equal(a.values.view(torch.int16), b.values.view(torch.int16)))
        native = same
        del native_cache, forward
    rows = []
    dim = key0.shape[-1]
    for i in range(n_layers):
        ours, theirs = output.layers[i], reference_output.layers[i]
        entry = {"layer": i,
                 "k": _north_star(ours.keys.index_select(2, index), theirs.keys.index_select(2, index), True),
                 "v": _north_star(ours.values.index_select(2, index), theirs.values.index_select(2, index)),
                 "attention": _north_star(attended[i].reshape(-1, dim), record["attention"][i].reshape(-1, dim))}
        for p, t in (("k", ours.keys), ("v", ours.values), ("attention", attended[i])):
            entry[p]["elements"] = len(positions) * (t.numel() // t.shape[2] if p != "attention" else
                                                     t.numel() // len(positions))
        if i + 1 < n_layers:
            entry["hidden_out_min_cos"] = row_errors(hidden_out[i].reshape(len(positions), -1),
                                                     record["inputs"][i + 1].reshape(len(positions), -1))["min_cos"]
        rows.append(entry)
    parts = ("k", "v", "attention")
    worst = {p: {"max_abs": max(r[p]["max_abs"] for r in rows), "min_cos": min(r[p]["min_cos"] for r in rows),
                 "beyond_2e-2": sum(r[p]["beyond_2e-2"] for r in rows),
                 "beyond_2e-2_within_2ulp": all(r[p]["beyond_2e-2_within_2ulp"] for r in rows),
                 "elements": sum(r[p]["elements"] for r in rows)} for p in parts}
    del output, cache, view
    return {"layers": rows, "worst": worst, "native_layer_call_bit_identical": native,
            "min_cos_all": min(worst[p]["min_cos"] for p in parts)}


def fp32_control(model, old):
    """The same model and stale cache in fp32 (bf16 values upcast exactly)."""
    from kv_cache_repair_amd.cache import cache_from_tensors

    control_model = copy.deepcopy(model).float()
    control_old = cache_from_tensors([(l.keys.float(), l.values.float()) for l in old.layers])
    return control_model, control_old


def parity_checks(model, shim, old, old_ids, new_ids, intervals, with_control=True) -> dict:
    positions = [p for s, e in intervals for p in range(s, e)]
    ours = hip_stage(shim, old, old_ids, new_ids, intervals)
    record = {}
    theirs = reference_stage(model, old, old_ids, new_ids, intervals, record=record)
    forced = teacher_forced_parity(model, new_ids, intervals, record, theirs)
    del record
    if with_control:
        control_model, control_old = fp32_control(model, old)
        control = reference_stage(control_model, control_old, old_ids, new_ids, intervals)
        del control_model, control_old
    else:
        control = theirs
    result = depth_parity(ours, theirs, control, positions)
    if not with_control:
        result.pop("precision_floor_gate_all_layers")
    result["layers"] = [{"layer": r["layer"], "part": r["part"], "gate": r["gate"],
                         "ours_vs_fp32_max_abs": r["ours_vs_fp32"]["max_abs"],
                         "reference_vs_fp32_max_abs": r["reference_vs_fp32"]["max_abs"]}
                        for r in result["layers"]] if with_control else []
    gate = all(r[p]["min_cos"] >= NORTH_STAR_MIN_COS and (r[p]["max_abs"] <= NORTH_STAR_MAX_ABS
                                                           or r[p]["beyond_2e-2_within_2ulp"])
               for r in forced["layers"] for p in ("k", "v", "attention"))
    result["teacher_forced_per_layer"] = {
        "method": "every layer fed the reference path's own input for it; its fresh K/V rows and attention output "
                  "against the reference layer's",
        "north_star_gate": gate, "worst": forced["worst"],
        "native_layer_call_bit_identical": forced["native_layer_call_bit_identical"],
        "per_layer_max_abs": [{p: round(r[p]["max_abs"], 6) for p in ("k", "v", "attention")}
                              for r in forced["layers"]]}
    del ours, theirs, control
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return result


# ----------------------------------------------------------------------------- kernel device timings
def graph_device_us(launch, per_graph: int = 20, replays: int = 5) -> float:
    """Device time of one ``launch`` (a raw libkvrepair call with bound
    arguments): ``per_graph`` back-to-back launches are captured in a graph, which
    is replayed ``replays`` times between two HIP events on the current stream,
    so no host time lies inside the measurement."""
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            launch()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1000.0 / (replays * per_graph)
    del graph
    return us


def launch_floor_us(device) -> float:
    """Per-launch device time of a one-element fill kernel timed like every
    libkvrepair call (graph of back-to-back launches): the floor under which
    no launch's average duration falls, whatever its bytes."""
    t = torch.zeros(1, device=device)
    return graph_device_us(lambda: t.zero_())


def _checked(fn, *args, after=()):
    """A launch of ``fn(*args, stream, *after)`` on the stream current at call
    time (a graph capture swaps it), raising on a nonzero status."""
    from kv_cache_repair_amd import _native

    def launch():
        status = fn(*args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), *after)
        if status != 0:
            raise RuntimeError(f"{fn.__name__} returned {status}: {_native.lib().kvr_status_string(status)}")
    return launch


def kernel_launchers(model, workload: Workload, old, old_ids, new_ids, device):
    """Raw libkvrepair calls with the stage's own shapes and layouts, arguments
    bound once: (launch, algorithmic bytes, flops or 0, launches per step)."""
    from kv_cache_repair_amd import _native
    from kv_cache_repair_amd.cache import build_halo_cache
    from kv_cache_repair_amd.kernels.indexed_attention import IndexedPlan

    w = workload
    lib = _native.lib()
    esz = 2
    code = _native.DTYPE_CODES[torch.bfloat16]
    positions = w.positions()
    b, n = len(positions), w.edited
    shim_model = SimpleNamespace(generator=model)
    shifted, _ = build_halo_cache(shim_model, old, old_ids, new_ids, 0)
    inv = model.model.rotary_emb.inv_freq.to(device=device, dtype=torch.float32).contiguous()
    out = {}

    # shift-cache build: prefix copy + rotated K tail + V tail, every layer, one launch
    olds_k = [l.keys for l in old.layers]
    olds_v = [l.values for l in old.layers]
    news_k = [l.keys for l in shifted.layers]
    news_v = [l.values for l in shifted.layers]
    s3o, s3n = _native.i64_array(_native.strides3(olds_k[0])), _native.i64_array(_native.strides3(news_k[0]))
    args = (_native.ptr_array(olds_k), _native.ptr_array(olds_v), _native.ptr_array(news_k),
            _native.ptr_array(news_v), len(olds_k), w.hkv, w.dim, w.dim, s3o, s3n, w.delete_at,
            w.delete_at + w.delete_span, w.delete_at, w.suffix, -w.delete_span, inv.data_ptr(), 1.0, code)
    out["kvr_shift_cache_build"] = (_checked(lib.kvr_shift_cache_build, *args),
                                    2 * 2 * w.layers * w.hkv * (w.delete_at + w.suffix) * w.dim * esz, 0, 1)

    # rotate only: the suffix K rows of every layer (BASELINE "rotate GB/s")
    keys = [k[:, :, w.delete_at + w.delete_span:] for k in olds_k]
    outs = [k[:, :, w.delete_at:] for k in news_k]
    args = (_native.ptr_array(keys), _native.ptr_array(outs), len(keys), w.hkv, w.suffix, w.dim, w.dim,
            _native.i64_array(_native.strides3(keys[0])), _native.i64_array(_native.strides3(outs[0])),
            -w.delete_span, inv.data_ptr(), 1.0, code)
    out["kvr_rope_delta_rotate"] = (_checked(lib.kvr_rope_delta_rotate, *args),
                                    2 * w.layers * w.hkv * w.suffix * w.dim * esz, 0, 0)

    # per-layer operators on layer 0 of the shifted cache, the stage's layouts:
    # fresh q/k/v as token-major transposed views, attention output [1, B, Hq, D]
    plan = IndexedPlan(positions, n).to(device)
    pos_ptr = plan.positions.data_ptr()
    cache_k, cache_v = news_k[0], news_v[0]
    gen = torch.Generator(device=device).manual_seed(5)
    qkv = torch.randn(1, b, (w.hq + 2 * w.hkv) * w.dim, device=device, generator=gen, dtype=torch.bfloat16)
    q = qkv[..., :w.hq * w.dim].view(1, b, w.hq, w.dim).transpose(1, 2)
    fk = qkv[..., w.hq * w.dim:(w.hq + w.hkv) * w.dim].view(1, b, w.hkv, w.dim).transpose(1, 2)
    fv = qkv[..., (w.hq + w.hkv) * w.dim:].view(1, b, w.hkv, w.dim).transpose(1, 2)
    q_out = torch.empty(1, b, w.hq, w.dim, device=device, dtype=torch.bfloat16).transpose(1, 2)
    cos, sin = model.model.rotary_emb(qkv, plan.positions.unsqueeze(0))
    cos, sin = cos.contiguous(), sin.contiguous()
    st18 = _native.i64_array(sum((_native.strides3(t) for t in (q, q_out, fk, fv, cache_k, cache_v)), []))
    cs = _native.i64_array([int(cos.stride(-2)), int(cos.stride(-1)), int(sin.stride(-2)), int(sin.stride(-1))])
    args = (q.data_ptr(), q_out.data_ptr(), fk.data_ptr(), fv.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(),
            cos.data_ptr(), sin.data_ptr(), pos_ptr, b, w.hq, w.hkv, n, w.dim, st18, cs, code)
    out["kvr_rope_scatter_kv"] = (_checked(lib.kvr_rope_scatter_kv, *args),
                                  (2 * (w.hq + 2 * w.hkv) + 2) * b * w.dim * esz, 0, w.layers)

    st12 = _native.i64_array(sum((_native.strides3(t) for t in (cache_k, cache_v, fk, fv)), []))
    args = (cache_k.data_ptr(), cache_v.data_ptr(), fk.data_ptr(), fv.data_ptr(), pos_ptr, b, w.hkv, n, w.dim, st12,
            code)
    out["kvr_indexed_scatter_kv"] = (_checked(lib.kvr_indexed_scatter_kv, *args),
                                     2 * 2 * w.hkv * b * w.dim * esz, 0, 0)

    # the packed executor's schedule: probabilities rounded to bf16 before PV, as its SDPA counterpart
    host, dev = plan.attention_schedule(w.hq, w.hkv, w.dim, torch.bfloat16, rounded=True)
    ws_bytes = int(lib.kvr_attention_workspace_bytes(host, len(host), w.hq, w.dim))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    attn_out = torch.empty(1, b, w.hq, w.dim, device=device, dtype=torch.bfloat16).permute(0, 2, 1, 3)
    st_attn = _native.i64_array(sum((_native.strides3(t) for t in (q, cache_k, cache_v, attn_out)), []))
    args = (q.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), attn_out.data_ptr(), pos_ptr, b, w.hq, w.hkv, n,
            w.dim, ctypes.c_float(w.dim ** -0.5), st_attn, dev.data_ptr(), len(host), host, ws.data_ptr(), ws_bytes,
            code)
    max_pos = max(positions)
    attn_bytes = (2 * b * w.hq * w.dim + 2 * w.hkv * (max_pos + 1) * w.dim) * esz
    attn_flops = 4 * w.hq * w.dim * sum(p + 1 for p in positions)
    out["kvr_packed_causal_attention"] = (_checked(lib.kvr_packed_causal_attention, *args), attn_bytes, attn_flops,
                                          w.layers)

    # projections of one layer as the stage's native forward launches them (<= 64 rows): q/k/v, o and down
    # leave their split-K partials to the consumer kernels (kvr_linear_multi_partials, no reduce launch),
    # gate/up runs with the SiLU gate in its epilogue (one split)
    if b <= 64:
        from kv_cache_repair_amd.kernels import projection as proj

        layer = model.model.layers[0]
        a, m = layer.self_attn, layer.mlp
        x = torch.randn(b, w.hidden, device=device, generator=gen, dtype=torch.bfloat16)
        xi = torch.randn(b, w.mlp, device=device, generator=gen, dtype=torch.bfloat16)
        xo = torch.randn(b, w.hq * w.dim, device=device, generator=gen, dtype=torch.bfloat16)
        calls, total_bytes = [], 0
        for weights, epi, xin in (
                ([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], proj.CONCAT, x),
                ([a.o_proj.weight], proj.CONCAT, xo),
                ([m.gate_proj.weight, m.up_proj.weight], proj.SILU_GATE, x),
                ([m.down_proj.weight], proj.CONCAT, xi)):
            pl = proj.ProjectionPlan(weights, epi)
            need = pl.workspace_bytes(b)
            wsp = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
            y = torch.empty(b, pl.n_out, device=device, dtype=torch.bfloat16)
            if epi == proj.SILU_GATE:
                launch = _checked(lib.kvr_linear_multi, xin.data_ptr(), pl._count, pl._w, pl._rows, pl._ldw,
                                  y.data_ptr(), b, pl.k, xin.stride(0), pl.n_out, epi, None, 0, wsp.data_ptr(), need,
                                  code)
                splits = None
            else:
                splits = ctypes.c_int32(0)
                launch = _checked(lib.kvr_linear_multi_partials, xin.data_ptr(), pl._count, pl._w, pl._rows,
                                  pl._ldw, y.data_ptr(), b, pl.k, xin.stride(0), pl.n_out, wsp.data_ptr(), need, code,
                                  after=(ctypes.byref(splits),))
            calls.append((launch, (xin, y, wsp, splits)))
            # algorithmic: the weights, x and the bf16 output once
            total_bytes += esz * (pl.rows * pl.k + b * pl.k + b * pl.n_out)
        keep = [c[1] for c in calls]

        def launch_all():
            for c, _ in calls:
                c()
        launch_all.keep = keep  # the bound tensors live as long as the launcher
        # one "launch" = the four projections of a layer; bytes/flops averaged per kvr_linear_multi call
        out["kvr_linear_multi"] = (launch_all, total_bytes, 0, 4 * w.layers, 4)
    else:
        # more rows than one kvr_linear_multi launch serves: the stage runs the modules' own
        # projections (torch -> hipBLASLt): one layer's seven GEMMs at the workload's row count
        layer = model.model.layers[0]
        a, m = layer.self_attn, layer.mlp
        x = torch.randn(b, w.hidden, device=device, generator=gen, dtype=torch.bfloat16)
        xi = torch.randn(b, w.mlp, device=device, generator=gen, dtype=torch.bfloat16)
        xo = torch.randn(b, w.hq * w.dim, device=device, generator=gen, dtype=torch.bfloat16)
        gemms = [(mod.weight.detach(), xin) for mod, xin in ((a.q_proj, x), (a.k_proj, x), (a.v_proj, x),
                                                             (a.o_proj, xo), (m.gate_proj, x), (m.up_proj, x),
                                                             (m.down_proj, xi))]
        outs = [torch.empty(b, wt.shape[0], device=device, dtype=torch.bfloat16) for wt, _ in gemms]

        def launch_gemms():
            for (wt, xin), y in zip(gemms, outs):
                torch.matmul(xin, wt.t(), out=y)
        launch_gemms.keep = (gemms, outs)
        params = sum(wt.numel() for wt, _ in gemms)
        nbytes = esz * (params + sum(xin.numel() + y.numel() for (_, xin), y in zip(gemms, outs)))
        # one "launch" = the seven GEMMs of a layer; per GEMM on average
        out["hipblaslt_projections"] = (launch_gemms, nbytes, 2 * b * params, 7 * w.layers, 7)
    launch_keep = (shifted, plan, qkv, q_out, cos, sin, ws, attn_out, host, dev)
    return out, launch_keep


def measure_kernels(model, workload, old, old_ids, new_ids, device) -> dict:
    launchers, keep = kernel_launchers(model, workload, old, old_ids, new_ids, device)
    kernels = {}
    for name, entry in launchers.items():
        launch, nbytes, flops, per_step = entry[:4]
        calls = entry[4] if len(entry) > 4 else 1
        us = graph_device_us(launch) / calls
        rec = {"avg_us": us, "algorithmic_bytes": nbytes / calls, "achieved_GBps": nbytes / calls / (us * 1e3),
               "frac_of_hbm_peak": nbytes / calls / (us * 1e3) / HBM_PEAK_GBPS, "launches_per_step": per_step,
               "total_us_per_step": us * per_step}
        if flops:
            rec["achieved_TFLOPs"] = flops / calls / (us * 1e6)
            rec["frac_of_bf16_mfma_peak"] = flops / calls / (us * 1e6) / MFMA_BF16_PEAK_TFLOPS
        kernels[name] = rec
    del keep
    torch.cuda.synchronize()
    return kernels


TRAFFIC_SUMMARIES = tuple(sorted((ROOT / "profiles").glob("*.md")))
KERNEL_SOURCES = {"kvr_packed_causal_attention": "kvr_attention.hip", "kvr_shift_cache_build": "kvr_rotate.hip",
                  "kvr_rope_delta_rotate": "kvr_rotate.hip", "kvr_indexed_scatter_kv": "kvr_scatter.hip",
                  "kvr_rope_scatter_kv": "kvr_fresh.hip", "kvr_linear_multi": "kvr_gemm.hip"}


def source_digest(name: str) -> str:
    import hashlib

    path = ROOT / "budgeted-kv-cache-repair_amd" / "csrc" / name
    return hashlib.sha256(path.read_bytes()).hexdigest()[:16]


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of ``kernel`` on ``workload`` from a committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's
    counts), or None when no summary covers it or it was measured on another
    version of the kernel source."""
    if kernel not in KERNEL_SOURCES:
        return None
    for summary in TRAFFIC_SUMMARIES:
        for line in summary.read_text().splitlines():
            if not line.startswith("traffic:"):
                continue
            fields = dict(item.partition("=")[::2] for item in line[len("traffic:"):].split())
            if (fields.get("kernel") == kernel and fields.get("workload", "c3") == workload
                    and fields.get("source_sha256") == source_digest(KERNEL_SOURCES[kernel])):
                return int(fields["bytes_per_launch"])
    return None


def rooflines(kernels: dict, workload: str) -> tuple[dict, dict]:
    """(roofline of the dominant kernel of the step, rooflines of the north-star kernels)."""
    def entry(name, bound="hbm"):
        k = kernels[name]
        if bound == "mfma":
            achieved, peak, unit = k["achieved_TFLOPs"], MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
        else:
            achieved, peak, unit = k["achieved_GBps"], HBM_PEAK_GBPS, "GB/s"
        return {"kernel": name, "bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                "frac": achieved / peak, "traffic": measured_traffic(name, workload), "avg_launch_us": k["avg_us"],
                "algorithmic_bytes_per_launch": k["algorithmic_bytes"]}

    stepping = {n: k for n, k in kernels.items() if k["launches_per_step"]}
    dominant = max(stepping, key=lambda n: stepping[n]["total_us_per_step"])
    attention_bound = "mfma" if workload in ("c4", "c5") else "hbm"
    # the bound of the dominant kernel: attention as above; hipBLASLt's projections of
    # more than 64 rows are MFMA-bound (2*rows flops per weight element read once)
    bound = {"kvr_packed_causal_attention": attention_bound, "hipblaslt_projections": "mfma"}.get(dominant, "hbm")
    north = {"rotate": entry("kvr_rope_delta_rotate"), "shift_cache_build": entry("kvr_shift_cache_build"),
             "scatter": entry("kvr_indexed_scatter_kv"), "fresh_row_epilogue": entry("kvr_rope_scatter_kv"),
             "attention": entry("kvr_packed_causal_attention", attention_bound)}
    north["attention"]["achieved_TFLOPs"] = kernels["kvr_packed_causal_attention"]["achieved_TFLOPs"]
    north["attention"]["achieved_GBps"] = kernels["kvr_packed_causal_attention"]["achieved_GBps"]
    return entry(dominant, bound), north


# ----------------------------------------------------------------------------- selection scoring
def reference_scores(embedding, ids, query):
    """The reference's chunked eager scorer (scoring.py:11-62) on the same GPU."""
    import torch.nn.functional as F

    device = ids.device
    q = F.normalize(embedding(torch.tensor([query], dtype=torch.long, device=device))[0].float(), dim=-1)
    scores = torch.full((ids.shape[0],), -float("inf"), dtype=torch.float32, device=device)
    exact = set(query)
    for start in range(0, ids.shape[0], 1024):
        chunk = ids[start:start + 1024]
        sim = torch.matmul(F.normalize(embedding(chunk).float(), dim=-1), q.transpose(0, 1)).max(dim=1).values
        boost = torch.tensor([0.25 if int(t) in exact else 0.0 for t in chunk.tolist()], dtype=torch.float32,
                             device=device)
        scores[start:start + chunk.shape[0]] = sim + boost
    return [float(v) for v in scores.tolist()]


def scoring_measurement(model, new_ids, device, launches=50, calls=10) -> dict:
    """Dense query relevance over the edited ids with the bench model's
    embedding table and a 12-token query (half of it taken from the prompt, so
    exact-id boosts occur): the kvr_query_relevance launch alone (HIP events on
    the launching stream), the Python API end to end (list of scores on the
    host), and the reference's eager scorer on the same GPU."""
    from kv_cache_repair_amd import _native
    from kv_cache_repair_amd.scoring import dense_query_relevance_scores

    embedding = model.get_input_embeddings()
    holder = SimpleNamespace(generator=model)  # the reference's scorer reads model.generator
    ids = new_ids[0]
    rng = random.Random(3)
    vocab = int(embedding.weight.shape[0])
    query = [int(ids[rng.randrange(ids.shape[0])]) for _ in range(6)] + [rng.randrange(vocab) for _ in range(6)]
    ours = lambda: dense_query_relevance_scores(model=holder, edited_input_ids=new_ids,  # noqa: E731
                                                query_token_ids=query)
    theirs = lambda: reference_scores(embedding, ids, query)  # noqa: E731
    got, _ = ours()
    want = theirs()
    max_abs = max(abs(a - b) for a, b in zip(got, want))

    table = embedding.weight
    lib = _native.lib()
    qd = torch.tensor(query, dtype=torch.long, device=device)
    out = torch.empty(ids.shape[0], dtype=torch.float32, device=device)
    launch = _checked(lib.kvr_query_relevance, table.data_ptr(), table.shape[0], table.stride(0), table.shape[1],
                      ids.data_ptr(), 0, ids.shape[0], qd.data_ptr(), len(query), ctypes.c_float(0.25),
                      out.data_ptr(), _native.DTYPE_CODES[table.dtype])
    kernel_us = graph_device_us(launch)
    n, hidden = ids.shape[0], table.shape[1]
    algorithmic = 2 * hidden * (n + len(query)) + 8 * n + 4 * n  # gathered rows, query rows, ids, scores
    return {"workload": f"edited ids ({n} tokens), embedding {tuple(table.shape)} bf16, {len(query)}-token query",
            "kernel_avg_us": kernel_us, "algorithmic_bytes": algorithmic,
            "achieved_GBps": algorithmic / (kernel_us * 1e3),
            "frac_of_peak": algorithmic / (kernel_us * 1e3) / HBM_PEAK_GBPS,
            "api_ms": time_steps(ours, calls, 2), "reference_same_gpu_ms": time_steps(theirs, calls, 2),
            "max_abs_vs_reference": max_abs}


# ----------------------------------------------------------------------------- CPU baselines
def _cpu_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_copy(model, workload: Workload, layers: int):
    """The first ``layers`` decoder layers of ``model`` (with its embedding, norm
    and head) as a CPU model holding the same weights bit for bit."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    cfg = copy.deepcopy(model.config)
    cfg.num_hidden_layers = layers
    if workload.family == "qwen3":
        cfg.layer_types = ["full_attention"] * layers
    ctor = Qwen3ForCausalLM if workload.family == "qwen3" else LlamaForCausalLM
    assert isinstance(cfg, (LlamaConfig, Qwen3Config))
    previous = torch.get_default_dtype()
    torch.set_default_dtype(next(model.parameters()).dtype)
    try:
        with torch.device("meta"):
            host = ctor(cfg)
    finally:
        torch.set_default_dtype(previous)
    host = host.to_empty(device="cpu").eval()
    source = dict(model.named_parameters())
    with torch.no_grad():
        for name, param in host.named_parameters():
            param.copy_(source[name])
        rotary = host.model.rotary_emb
        rotary.inv_freq = model.model.rotary_emb.inv_freq.detach().cpu()
        rotary.original_inv_freq = rotary.inv_freq.clone()
        rotary.attention_scaling = model.model.rotary_emb.attention_scaling
    host.set_attn_implementation("sdpa")
    return host


def cpu_baseline(workload: Workload, model, old, old_ids, new_ids, layers_sample: int = 0,
                 repeats: int = 5) -> dict:
    """The oracle's torch restatement of the reference stage (rotate chain +
    packed SDPA forward) on every host core, over a host copy of the GPU run's
    own model and stale cache: all layers by default (``layers_sample`` > 0 times
    only the first layers and scales), median of ``repeats`` runs after one
    warm-up."""
    from kv_cache_repair_amd.cache import cache_from_tensors
    from oracle import reference_path as ref

    layers_sample = workload.layers if layers_sample <= 0 else min(layers_sample, workload.layers)
    threads = max(1, os.cpu_count() or 1)
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        t_copy = time.perf_counter()
        model = host_copy(model, workload, layers_sample)
        old = cache_from_tensors([(l.keys.cpu(), l.values.cpu()) for l in old.layers[:layers_sample]])
        old_ids, new_ids = old_ids.cpu(), new_ids.cpu()
        copy_s = time.perf_counter() - t_copy
        intervals = workload.intervals()
        ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)  # warm-up (allocator, kernels)
        samples = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)
            samples.append((time.perf_counter() - t0) * 1000.0)
        per_sample_ms = statistics.median(samples)
        del model, old
    finally:
        torch.set_num_threads(previous)
    scale = workload.layers / layers_sample
    scope = (f"all {workload.layers} layers" if scale == 1 else
             f"the first {layers_sample} of {workload.layers} layers, scaled x{scale:g}")
    return {"value": per_sample_ms * scale, "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"oracle torch restatement of the reference stage (eager rotate chain, clone, boolean mask, "
                      f"index_copy_, HF sdpa) over {scope} of the {workload.name} workload on a host copy of the "
                      f"GPU run's model and stale cache, bf16, median of {repeats} runs after one warm-up; torch "
                      f"threads = os.cpu_count()",
            "samples_ms": samples, "host_copy_s": copy_s, "cpu": _cpu_name(), "os_cpu_count": os.cpu_count()}


def cpu_kernel_baseline(workload: Workload, repeats: int = 2) -> dict:
    """The three north-star steps the reference way (eager rotate chain,
    index_copy_ pair, repeat_kv + masked SDPA) on every host core, for one layer
    of the workload (attention over ``heads`` query heads of one KV group where
    a full layer would take minutes), scaled to the whole step: bounded
    samples for configs whose full CPU stage is impractical."""
    from oracle import reference_path as ref

    w = workload
    threads = max(1, os.cpu_count() or 1)
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(w.seed)
    try:
        inv = 1.0 / (w.theta ** (torch.arange(0, w.dim, 2, dtype=torch.float32) / w.dim))
        tail = torch.randn(1, w.hkv, w.suffix, w.dim, generator=gen).to(torch.bfloat16)
        shift = -w.delete_span

        def rotate():
            freqs = inv[None, :] * float(shift)
            emb = torch.cat((freqs, freqs), dim=-1)
            cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
            return tail * cos + ref.rotate_half(tail) * sin

        positions = torch.tensor(w.positions(), dtype=torch.long)
        b = positions.numel()
        cache_k = torch.randn(1, w.hkv, w.edited, w.dim, generator=gen).to(torch.bfloat16)
        cache_v = torch.randn(1, w.hkv, w.edited, w.dim, generator=gen).to(torch.bfloat16)
        fresh = torch.randn(1, w.hkv, b, w.dim, generator=gen).to(torch.bfloat16)

        def scatter():
            cache_k.index_copy_(2, positions, fresh)
            cache_v.index_copy_(2, positions, fresh)

        group = w.hq // w.hkv
        heads = group if b * w.edited > 64 * 8192 else w.hq  # one KV group for the large configs
        q = torch.randn(1, heads, b, w.dim, generator=gen).to(torch.bfloat16)
        kv_heads = heads // group
        mask = (torch.arange(w.edited)[None, :] <= positions[:, None])[None, None]

        def attention():
            k = cache_k[:, :kv_heads].repeat_interleave(group, dim=1)
            v = cache_v[:, :kv_heads].repeat_interleave(group, dim=1)
            return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)

        def timed(fn):
            fn()
            samples = []
            for _ in range(repeats):
                t0 = time.perf_counter()
                fn()
                samples.append((time.perf_counter() - t0) * 1000.0)
            return statistics.median(samples)

        rot_ms, sc_ms, at_ms = timed(rotate), timed(scatter), timed(attention)
    finally:
        torch.set_num_threads(previous)
    return {"cores": threads, "cpu": _cpu_name(), "kind": "port", "repeats": repeats,
            "rotate_ms_per_step": rot_ms * w.layers, "scatter_ms_per_step": sc_ms * w.layers,
            "attention_ms_per_step": at_ms * w.layers * (w.hq / heads),
            "sample": f"one layer of {w.name} per op on the host CPU (bf16, eager torch as the reference runs it: "
                      f"rotate chain over {w.hkv}x{w.suffix} rows, index_copy_ K/V of {b} rows, repeat_kv + "
                      f"masked SDPA over {heads} of {w.hq} query heads), median of {repeats} after a warm-up, "
                      f"scaled to {w.layers} layers and {w.hq} heads"}


# ----------------------------------------------------------------------------- reference benchmark grid
def selected_intervals(length: int, budget: int, count: int) -> list[tuple[int, int]]:
    """The reference benchmark's support geometry (benchmark_refresh.py:35-49):
    ``count`` intervals of budget/count rows placed symmetrically about the
    context middle, so the causal pair count is the same for every count."""
    if length <= 0 or budget <= 0 or count <= 0 or budget % count:
        raise ValueError("length and budget must be positive; budget must be divisible by interval count")
    width = budget // count
    if count == 1:
        starts = [(length - width) // 2]
    else:
        starts = [round(length / 4 + i * length / (2 * (count - 1)) - width / 2) for i in range(count)]
    intervals = [(s, s + width) for s in starts]
    if intervals[0][0] < 0 or intervals[-1][1] > length:
        raise ValueError("selected support does not fit the sequence")
    if any(a[1] >= b[0] for a, b in zip(intervals, intervals[1:])):
        raise ValueError("intervals must be separated; increase length or reduce budget/count")
    return intervals


def _interleave(calls, names, samples, rng, repeats):
    for _ in range(repeats):
        order = names.copy()
        rng.shuffle(order)
        for name in order:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = calls[name]()
            torch.cuda.synchronize()
            samples[name].append((time.perf_counter() - t0) * 1000.0)
            del out


def interleaved_latency(calls: dict, warmups: int, repeats: int, seed: int) -> dict:
    """Per-call wall time of each entry of ``calls``, each call bracketed by
    ``torch.cuda.synchronize()``: ``warmups`` untimed rounds, then ``repeats``
    rounds that run every entry once in a shuffled order (benchmark_refresh.py:
    100-126). Returns {name: median/mean/p95 and the raw samples, in ms}."""
    names = list(calls)
    for _ in range(warmups):
        for name in names:
            calls[name]()
            torch.cuda.synchronize()
    samples = {name: [] for name in names}
    rng = random.Random(seed)
    with no_gc():
        _interleave(calls, names, samples, rng, repeats)

    def summary(values):
        ordered = sorted(values)
        return {"median_ms": statistics.median(values), "mean_ms": statistics.mean(values),
                "p95_ms": ordered[math.ceil(0.95 * len(ordered)) - 1], "raw_ms": values}

    return {name: summary(v) for name, v in samples.items()}


def reference_sequential(model, shifted, ids, intervals):
    """The reference's sequential schedule on this GPU (execution.py:34-59 over
    cache.py:147-192): per interval a clone of every layer's prefix, the native
    forward over the interval's tokens, then a new cache concatenated from the
    old rows before, the fresh rows and the old rows after."""
    from kv_cache_repair_amd.cache import cache_from_tensors

    cache = shifted
    for start, end in intervals:
        prefix = cache_from_tensors([(l.keys[:, :, :start].clone(), l.values[:, :, :start].clone())
                                     for l in cache.layers])
        mask = torch.ones((1, end), dtype=torch.long, device=ids.device)
        fresh = model.model(input_ids=ids[:, start:end], attention_mask=mask, past_key_values=prefix, use_cache=True,
                            return_dict=True).past_key_values
        cache = cache_from_tensors([
            (torch.cat((o.keys[:, :, :start], f.keys[:, :, start:end], o.keys[:, :, end:]), dim=2),
             torch.cat((o.values[:, :, :start], f.values[:, :, start:end], o.values[:, :, end:]), dim=2))
            for o, f in zip(cache.layers, fresh.layers)])
    return cache


def grid_case(model, length: int, count: int, budget: int, warmups: int, repeats: int, seed: int) -> dict:
    """One case of the reference grid: a stale cache of ``length + 8`` tokens (K/V
    ~ N(0,1)) loses 8 tokens at length // 8 and is shifted (untimed); then the
    packed refresh alone (ownership copy, plan upload, layer-major forward) is
    timed for this build and for the reference path, interleaved in shuffled
    order (benchmark_refresh.py:52-61, 106-126). The reference benchmark's
    sequential schedule is timed beside them: this build's sequential executor
    against the reference's sequential schedule, which it must equal bit for
    bit (benchmark_refresh.py:150-153)."""
    from kv_cache_repair_amd.cache import OperatorShim, build_halo_cache, cache_from_tensors
    from kv_cache_repair_amd.execution import sequential_repair
    from kv_cache_repair_amd.kernels.packed_cache import packed_interval_repair

    device = model.device
    w = WORKLOADS["c3"]
    gen = torch.Generator(device=device).manual_seed(seed)
    old = cache_from_tensors([(torch.randn(1, w.hkv, length + 8, w.dim, device=device, generator=gen,
                                           dtype=torch.bfloat16),
                               torch.randn(1, w.hkv, length + 8, w.dim, device=device, generator=gen,
                                           dtype=torch.bfloat16)) for _ in range(w.layers)])
    old_ids = torch.randint(4, w.vocab, (1, length + 8), device=device, generator=gen)
    at = length // 8
    old_ids[0, at] = (old_ids[0, at + 8] + 1) % w.vocab
    ids = torch.cat((old_ids[:, :at], old_ids[:, at + 8:]), dim=1)
    shim = OperatorShim(model)
    shifted, alignment = build_halo_cache(shim, old, old_ids, ids, 0)
    intervals = selected_intervals(length, budget, count)
    positions = [p for s, e in intervals for p in range(s, e)]
    calls = {"hip": lambda: packed_interval_repair(shim, shifted, ids, intervals)[0],
             "reference_packed_sdpa": lambda: reference_stage(model, None, None, ids, intervals, shifted=shifted),
             "sequential": lambda: sequential_repair(shim, shifted, ids, intervals)[0],
             "reference_sequential": lambda: reference_sequential(model, shifted, ids, intervals)}
    outputs = {name: fn() for name, fn in calls.items()}
    index = torch.tensor(positions, device=device)

    def max_abs_rows(x, y):
        return max((a.index_select(2, index).float() - b.index_select(2, index).float()).abs().max().item()
                   for la, lb in zip(x.layers, y.layers) for a, b in ((la.keys, lb.keys), (la.values, lb.values)))

    def bitwise(x, y):
        return all(torch.equal(a.view(torch.int16), b.view(torch.int16))
                   for la, lb in zip(x.layers, y.layers) for a, b in ((la.keys, lb.keys), (la.values, lb.values)))

    max_abs = max_abs_rows(outputs["hip"], outputs["reference_packed_sdpa"])
    same_schedule = {name: {"bitwise_equal": bitwise(outputs[name], outputs["reference_sequential"]),
                            "max_abs": max_abs_rows(outputs[name], outputs["reference_sequential"])}
                     for name in ("sequential",)}
    packed_vs_sequential = max_abs_rows(outputs["hip"], outputs["reference_sequential"])
    del outputs
    lat = interleaved_latency(calls, warmups, repeats, seed)
    return {"metric": "refresh-only latency (ms), reference benchmark grid", "length": length,
            "interval_count": count, "token_budget": budget, "intervals": intervals,
            "causal_query_key_pairs": sum(p + 1 for p in positions), "position_shift": alignment["position_shift"],
            "value": lat["hip"]["median_ms"], "unit": "ms", "higher_is_better": False,
            "reference_same_gpu_ms": lat["reference_packed_sdpa"]["median_ms"],
            "speedup": lat["reference_packed_sdpa"]["median_ms"] / lat["hip"]["median_ms"],
            "sequential_ms": lat["sequential"]["median_ms"],
            "reference_sequential_ms": lat["reference_sequential"]["median_ms"],
            "same_schedule_vs_reference_sequential": same_schedule,
            "packed_max_abs_vs_reference_sequential": packed_vs_sequential,
            "latency": lat, "max_abs_vs_reference": max_abs, "warmups": warmups, "repeats": repeats, "seed": seed,
            "scope": "refresh only (ownership copy, plan upload, packed forward); the shift is untimed as in the "
                     "reference benchmark", "dtype": "bf16",
            "data": "synthetic (random-init 8B-shaped Llama, K/V ~ N(0,1), random ids)"}


# ----------------------------------------------------------------------------- main
def profile_kernels(args, workload: Workload, device) -> dict:
    """Launch the named libkvrepair calls (kernel_launchers' names, or "all")
    with the stage's shapes, eagerly and synchronised one by one: a short
    program for rocprofv3 counter passes, without the stage or its checks."""
    from kv_cache_repair_amd import _native

    _native.lib()
    model = make_model(device, workload)
    old, old_ids, new_ids = make_request(device, workload)
    launchers, keep = kernel_launchers(model, workload, old, old_ids, new_ids, device)
    names = sorted(launchers) if args.profile_kernels == "all" else args.profile_kernels.split(",")
    unknown = [n for n in names if n not in launchers]
    if unknown:
        raise SystemExit(f"unknown kernel(s) {unknown}; choose from {sorted(launchers)}")
    for name in names:
        for _ in range(args.profile_launches):
            launchers[name][0]()
            torch.cuda.synchronize()
    del keep
    return {"profiled": names, "launches_each": args.profile_launches, "workload": workload.name}


def host_timeline(args, workload: Workload, device) -> dict:
    """When, within one synchronised stage call, the host issues the stage's
    three launches that bracket its host work: the shift-cache build, the
    refresh's first kernel (kvr_refresh_inputs) and the enqueue of every layer
    (kvr_decoder_forward, entry and return), plus the call's return and its
    completion (after torch.cuda.synchronize()). Medians over ``args.steps``
    calls after ``args.warmup``, microseconds from the call's entry. The GPU
    idles until the first launch and between the build's end and the refresh's
    first kernel whenever the host work between them outlasts the build."""
    from kv_cache_repair_amd import _native
    from kv_cache_repair_amd.cache import OperatorShim

    lib = _native.lib()
    model = make_model(device, workload)
    shim = OperatorShim(model)
    old, old_ids, new_ids = make_request(device, workload)
    intervals = workload.intervals()
    host_ids = (old_ids.cpu(), new_ids.cpu())
    marks = {}
    originals = {}

    def stamped(name):
        fn = originals[name] = getattr(lib, name)

        def call(*a):
            marks[name + " entry"] = time.perf_counter()
            status = fn(*a)
            marks[name + " return"] = time.perf_counter()
            return status
        return call

    names = ("kvr_shift_cache_build", "kvr_refresh_inputs", "kvr_decoder_forward")
    for name in names:
        setattr(lib, name, stamped(name))
    samples = []
    try:
        with no_gc():
            for i in range(args.warmup + args.steps):
                marks.clear()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                out = hip_stage(shim, old, old_ids, new_ids, intervals, host_ids=host_ids)
                t1 = time.perf_counter()
                torch.cuda.synchronize()
                t2 = time.perf_counter()
                del out
                if i >= args.warmup:
                    samples.append({**{k: (v - t0) * 1e6 for k, v in marks.items()},
                                    "stage call returns": (t1 - t0) * 1e6, "stage complete (synchronised)": (t2 - t0) * 1e6})
    finally:
        for name, fn in originals.items():
            setattr(lib, name, fn)
    keys = sorted(samples[0], key=lambda k: statistics.median(s[k] for s in samples))
    # the launchers hold raw pointers into `keep`'s tensors (the build's output
    # cache among them): keep them alive until the timing is done
    launchers, keep = kernel_launchers(model, workload, old, old_ids, new_ids, device)
    build_us = graph_device_us(launchers["kvr_shift_cache_build"][0])
    del launchers, keep
    torch.cuda.synchronize()
    return {"metric": "host timeline of one synchronised stage call (us from entry, medians)",
            "workload": workload.description, "calls": args.steps, "warmup": args.warmup,
            "timeline_us": {k: round(statistics.median(s[k] for s in samples), 1) for k in keys},
            "kernel_device_us": {"kvr_shift_cache_build": build_us}}


def run_workload(args, workload: Workload, device) -> dict:
    from kv_cache_repair_amd import _native
    from kv_cache_repair_amd.cache import OperatorShim

    _native.lib()
    model = make_model(device, workload)
    shim = OperatorShim(model)
    old, old_ids, new_ids = make_request(device, workload)
    intervals = workload.intervals()
    headline = workload.name == "c3"

    # correctness gate (untimed): rotated/copied rows bit-exact, refreshed rows against
    # the reference path and an fp32 control at every layer
    checks = {} if args.no_reference else parity_checks(model, shim, old, old_ids, new_ids, intervals,
                                                        with_control=not args.no_fp32_control)

    host_ids = (old_ids.cpu(), new_ids.cpu())
    step = lambda: hip_stage(shim, old, old_ids, new_ids, intervals, host_ids=host_ids)  # noqa: E731
    per_call = time_calls(step, args.steps, args.warmup)
    ms = per_call["median_ms"]
    back_to_back = time_steps(step, args.steps, 0)
    kernels = measure_kernels(model, workload, old, old_ids, new_ids, device)
    roofline, north = rooflines(kernels, workload.name)
    floor_us = launch_floor_us(device)

    reference = None
    interleaved = None
    if not args.no_reference:
        ref_step = lambda: reference_stage(model, old, old_ids, new_ids, intervals)  # noqa: E731
        ref_calls = time_calls(ref_step, args.steps, max(1, args.warmup))
        ref_ms = ref_calls["median_ms"]
        reference = {"ms_per_step": ref_ms, "p95_ms": ref_calls["p95_ms"], "speedup": ref_ms / ms,
                     "back_to_back_ms_per_step": time_steps(ref_step, args.steps, 0),
                     "what": "reference eager path on the same GPU: per-layer rotate chain + cats, clone_cache, "
                             "bool mask, index_copy_, HF sdpa_attention_forward with repeat_kv",
                     "sdpa": sdpa_backend_used(ref_step)}
        if args.interleaved_repeats > 0:
            lat = interleaved_latency({"hip": step, "reference_same_gpu": ref_step}, args.interleaved_warmups,
                                      args.interleaved_repeats, 71)
            interleaved = {"warmups": args.interleaved_warmups, "repeats": args.interleaved_repeats, "seed": 71,
                           "speedup_median": lat["reference_same_gpu"]["median_ms"] / lat["hip"]["median_ms"],
                           "latency": lat,
                           "method": "each call bracketed by torch.cuda.synchronize(), both paths once per round in "
                                     "a shuffled order"}
    scoring = scoring_measurement(model, new_ids, device) if headline else None
    if args.no_cpu_baseline:
        cpu = None
    elif headline:
        cpu = cpu_baseline(workload, model, old, old_ids, new_ids, args.cpu_layers)
    else:
        cpu = cpu_kernel_baseline(workload)
    del old
    suffix = workload.suffix
    rotate = kernels["kvr_rope_delta_rotate"]
    line = {
        "metric": METRIC if headline else f"refresh-stage latency (ms) per repair, {workload.name}",
        "value": ms, "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "p95_ms": per_call["p95_ms"], "back_to_back_ms_per_step": back_to_back,
        "timing": "value = ms_per_step = median of the steps' per-call samples, each call bracketed by "
                  "torch.cuda.synchronize() (benchmark_refresh.py:106-126); back_to_back_ms_per_step = the same "
                  "steps run back to back between two synchronisations",
        "per_call_samples_ms": per_call["samples_ms"],
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init model of the workload's shape, K/V ~ N(0,1), random ids)",
        "config": {"workload": workload.description, "layers": workload.layers, "kv_heads": workload.hkv,
                   "q_heads": workload.hq, "head_dim": workload.dim, "cache_tokens": workload.total,
                   "edited_tokens": workload.edited, "suffix_rows": suffix, "shift": -workload.delete_span,
                   "budget_rows": len(workload.positions()),
                   "intervals": intervals if len(intervals) <= 16 else f"{len(intervals)} intervals"},
        "rotate_GBps": rotate["achieved_GBps"],
        "rotate": {"avg_us": rotate["avg_us"], "algorithmic_bytes": rotate["algorithmic_bytes"],
                   "frac_of_peak": rotate["frac_of_hbm_peak"]},
        "roofline": roofline, "rooflines": north, "kernels": kernels,
        "kernel_timing": "HIP events around 5 replays of a graph of 20 back-to-back launches of each libkvrepair "
                         "call with the stage's shapes (device time only); kvr_linear_multi = one layer's four "
                         "projections as the native forward launches them (q/k/v, o, down leave split-K partials "
                         "to their consumers: kvr_linear_multi_partials), per projection",
        "launch_floor_us": floor_us,
        "launch_floor": "the same graph timing of a one-element fill kernel: the per-launch time no launch "
                        "goes below (small launches, such as the scatter and the epilogue at <= 64 rows, sit near it)",
        "reference_same_gpu": reference, "interleaved": interleaved, "checks": checks, "selection_scoring": scoring,
        "cpu_baseline": cpu, "device": torch.cuda.get_device_name(device),
    }
    return line


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="c3",
                        help="BASELINE configuration (c3 is the headline; others print a secondary line)")
    parser.add_argument("--grid", action="store_true", help="the reference benchmark's grid (one line per case)")
    parser.add_argument("--grid-repeats", type=int, default=20)
    parser.add_argument("--grid-warmups", type=int, default=10)
    parser.add_argument("--interleaved-repeats", type=int, default=20,
                        help="rounds of per-call timing, this build and the reference stage in shuffled order "
                             "(0 skips); reported beside the bracketed value, which it does not change")
    parser.add_argument("--interleaved-warmups", type=int, default=10)
    parser.add_argument("--cpu-layers", type=int, default=0,
                        help="layers in the CPU-baseline sample (0: all layers of the workload)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-reference", action="store_true", help="skip the same-GPU reference stage and checks")
    parser.add_argument("--no-fp32-control", action="store_true", help="parity checks without the fp32 control")
    parser.add_argument("--calibration-copy-mib", type=int, default=0,
                        help="after the run, copy a buffer of this many MiB three times with a plain device-to-device "
                             "copy (the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counts)")
    parser.add_argument("--profile-kernels", default="",
                        help="comma-separated libkvrepair calls (or 'all') to launch --profile-launches times each "
                             "with the workload's shapes, for rocprofv3 counter passes; no stage timing")
    parser.add_argument("--profile-launches", type=int, default=5)
    parser.add_argument("--host-timeline", action="store_true",
                        help="print when one synchronised stage call issues its key launches (no stage timing)")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build runs on a single GPU (--gpus {args.gpus} requested). "
              f"Multi-GPU sharding is a design note only.", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0:
        parser.error("steps must be positive and warmup nonnegative")
    if not torch.cuda.is_available():
        parser.error("bench.py needs a GPU")
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.grid:
        from kv_cache_repair_amd import _native

        _native.lib()
        model = make_model(device, C3)
        for length in (2048, 8192):
            for count in (1, 4, 16):
                print(json.dumps(grid_case(model, length, count, 64, args.grid_warmups, args.grid_repeats, 71)),
                      flush=True)
        return 0
    if args.host_timeline:
        line = host_timeline(args, WORKLOADS[args.workload], device)
    elif args.profile_kernels:
        line = profile_kernels(args, WORKLOADS[args.workload], device)
    else:
        line = run_workload(args, WORKLOADS[args.workload], device)
    print(json.dumps(line), flush=True)
    if args.calibration_copy_mib > 0:
        src = torch.empty(args.calibration_copy_mib << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
