"""Torch restatement of the reference's eager refresh path — TEST INFRASTRUCTURE ONLY.

The reference (yh0903/budgeted-kv-cache-repair) pins transformers 4.57.6 and
cannot run on the installed transformers 5.15.0. This module restates its
default path op for op on 5.15 so tests have the reference's own numerics to
compare against, on CPU or on the GPU:

* rotate:   shifted_suffix_keys (cache.py:47-77) — HF rotary_emb at
  position=shift, cast to the key dtype, key*cos + rotate_half(key)*sin;
* shift cache: build_halo_cache (cache.py:103-144) with clone/cat per layer;
* packed refresh: packed_interval_repair with attention_backend="sdpa",
  writeback_backend="torch" (kernels/packed_cache.py:225-298): clone_cache,
  boolean mask key <= position (:205-207), per-layer index_copy_ (:189-191),
  HF sdpa_attention_forward with repeat_kv (:60-67);
* sequential interval recurrence (execution.py:34-59, cache.py:147-192).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
it; the product package never imports it.
"""

from __future__ import annotations

import copy
import threading

import torch
from transformers.cache_utils import Cache, DynamicCache, DynamicLayer

_NAME = "oracle_reference_packed_sdpa"
_LOCK = threading.Lock()


def base_model(model):
    return getattr(model, "base_model", model)


def layer_kv(cache, index):
    layer = cache.layers[index]
    return layer.keys, layer.values


def cache_from_tensors(pairs) -> DynamicCache:
    """A DynamicCache whose layers hold exactly the given tensors (no copy)."""
    cache = DynamicCache()
    for key, value in pairs:
        layer = DynamicLayer()
        layer.keys, layer.values = key, value
        layer.dtype, layer.device = key.dtype, key.device
        layer.is_initialized = True
        cache.layers.append(layer)
    return cache


def rotate_half(x):
    """cache.py:25-28: [x1, x2] -> [-x2, x1]."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def clone_cache(cache, length=None) -> DynamicCache:
    """cache.py:31-44."""
    out = []
    for i in range(len(cache.layers)):
        k, v = layer_kv(cache, i)
        end = k.shape[2] if length is None else int(length)
        out.append((k[:, :, :end].clone(), v[:, :, :end].clone()))
    return cache_from_tensors(out)


@torch.no_grad()
def shifted_suffix_keys(model, key, shift):
    """cache.py:47-77, eager op for op."""
    if not key.shape[2] or not shift:
        return key.clone()
    base = base_model(model)
    positions = torch.full((1, key.shape[2]), int(shift), dtype=torch.long, device=key.device)
    cos, sin = base.rotary_emb(key, positions)
    cos = cos.unsqueeze(1).to(device=key.device, dtype=key.dtype)
    sin = sin.unsqueeze(1).to(device=key.device, dtype=key.dtype)
    rotary_dim = cos.shape[-1]
    if rotary_dim >= key.shape[-1]:
        return key * cos + rotate_half(key) * sin
    rotated = key[..., :rotary_dim]
    rotated = rotated * cos + rotate_half(rotated) * sin
    return torch.cat((rotated, key[..., rotary_dim:]), dim=-1)


@torch.no_grad()
def run_tokens_from_prefix(model, prefix_cache, input_ids, end_position):
    """cache.py:80-100."""
    if not input_ids.shape[1]:
        return prefix_cache
    mask = torch.ones((1, int(end_position)), dtype=torch.long, device=input_ids.device)
    return base_model(model)(input_ids=input_ids, attention_mask=mask, past_key_values=prefix_cache,
                             use_cache=True, return_dict=True).past_key_values


def token_alignment(old_ids, new_ids):
    """alignment.py:21-31 (lists of ints)."""
    prefix = 0
    while prefix < min(len(old_ids), len(new_ids)) and old_ids[prefix] == new_ids[prefix]:
        prefix += 1
    maximum = min(len(old_ids) - prefix, len(new_ids) - prefix)
    suffix = 0
    while suffix < maximum and old_ids[-1 - suffix] == new_ids[-1 - suffix]:
        suffix += 1
    return {
        "prefix": prefix,
        "suffix": suffix,
        "old_suffix_start": len(old_ids) - suffix,
        "new_suffix_start": len(new_ids) - suffix,
        "mandatory_changed_tokens": len(new_ids) - prefix - suffix,
        "position_shift": (len(new_ids) - suffix) - (len(old_ids) - suffix),
    }


@torch.no_grad()
def build_halo_cache(model, old_cache, old_ids, new_ids, halo_tokens=0):
    """cache.py:103-144."""
    align = token_alignment([int(x) for x in old_ids[0].tolist()], [int(x) for x in new_ids[0].tolist()])
    halo = min(max(int(halo_tokens), 0), align["suffix"])
    recompute_end = align["new_suffix_start"] + halo
    prefix_cache = clone_cache(old_cache, align["prefix"])
    recomputed = run_tokens_from_prefix(model, prefix_cache, new_ids[:, align["prefix"]:recompute_end],
                                        recompute_end)
    old_tail_start = align["old_suffix_start"] + halo
    out = []
    for i in range(len(old_cache.layers)):
        ek, ev = layer_kv(recomputed, i)
        ok, ov = layer_kv(old_cache, i)
        tail_k = shifted_suffix_keys(model, ok[:, :, old_tail_start:], align["position_shift"])
        tail_v = ov[:, :, old_tail_start:].clone()
        out.append((torch.cat((ek[:, :, :recompute_end], tail_k), dim=2),
                    torch.cat((ev[:, :, :recompute_end], tail_v), dim=2)))
    return cache_from_tensors(out), {**align, "halo_tokens": halo,
                                     "recomputed_tokens": align["mandatory_changed_tokens"] + halo}


@torch.no_grad()
def repair_window(model, base_cache, ids, start, end):
    """cache.py:147-192."""
    if end <= start:
        return base_cache
    prefix = clone_cache(base_cache, start)
    recomputed = run_tokens_from_prefix(model, prefix, ids[:, start:end], end)
    out = []
    for i in range(len(base_cache.layers)):
        ok, ov = layer_kv(base_cache, i)
        nk, nv = layer_kv(recomputed, i)
        out.append((torch.cat((ok[:, :, :start], nk[:, :, start:end], ok[:, :, end:]), dim=2),
                    torch.cat((ov[:, :, :start], nv[:, :, start:end], ov[:, :, end:]), dim=2)))
    return cache_from_tensors(out)


@torch.no_grad()
def sequential_repair(model, base_cache, ids, intervals):
    """execution.py:34-59: one forward per interval, in causal order."""
    cache = base_cache
    for start, end in intervals:
        cache = repair_window(model, cache, ids, start, end)
    return cache


# ---------------------------------------------------------------------------
# packed executor with SDPA attention and torch index_copy_ writeback
# ---------------------------------------------------------------------------
def _sdpa_packed(module, query, key, value, attention_mask, *, scaling=None, dropout=0.0,
                 oracle_packed_mask=None, oracle_record=None, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    out, weights = sdpa_attention_forward(module, query, key, value, oracle_packed_mask, dropout=0.0,
                                          scaling=scaling, is_causal=False)
    if oracle_record is not None:  # [1, B, Hq, D], the o_proj input
        oracle_record["attention"][module.layer_idx] = out.detach().clone()
    return out, weights


def _register():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    with _LOCK:
        if _NAME not in ALL_ATTENTION_FUNCTIONS:
            ALL_ATTENTION_FUNCTIONS.register(_NAME, _sdpa_packed)


class _IndexCopyLayer(DynamicLayer):
    def __init__(self, key, value, positions):
        super().__init__()
        self.keys, self.values = key, value
        self.dtype, self.device = key.dtype, key.device
        self.is_initialized = True
        self._positions = positions

    def update(self, key_states, value_states, *args, **kwargs):
        self.keys.index_copy_(2, self._positions, key_states)
        self.values.index_copy_(2, self._positions, value_states)
        return self.keys, self.values

    def get_mask_sizes(self, query_length):
        return self.keys.shape[2], 0


def _recording_forward(forward, index, record):
    """A decoder layer's forward that first records its input hidden rows (and,
    at layer 0, the rotary tables the model computed for the selected rows)."""
    def run(hidden_states, *args, **kwargs):
        record["inputs"][index] = hidden_states.detach().clone()
        if index == 0:
            record["tables"] = tuple(t.detach().clone() for t in kwargs["position_embeddings"])
        return forward(hidden_states, *args, **kwargs)
    return run


def _view_with_attention(base, name):
    config = copy.deepcopy(base.config)
    config._attn_implementation = name
    view = copy.copy(base)
    view._modules = base._modules.copy()
    view.config = config
    layers = []
    for original in base.layers:
        layer = copy.copy(original)
        layer._modules = original._modules.copy()
        attention = copy.copy(original.self_attn)
        attention._modules = original.self_attn._modules.copy()
        attention.config = config
        layer._modules["self_attn"] = attention
        layers.append(layer)
    view._modules["layers"] = torch.nn.ModuleList(layers)
    return view


@torch.no_grad()
def packed_sdpa_repair(model, base_cache, ids, intervals, record=None):
    """packed_cache.py:225-298 with the default sdpa/torch backends.

    ``record`` (a dict) receives, per decoder layer, what teacher-forced
    per-layer checks need: ``inputs[i]`` the layer's input hidden rows,
    ``attention[i]`` its attention output (the o_proj input, [1, B, Hq, D]),
    and ``tables`` the (cos, sin) rotary tables of the selected rows."""
    selected = [p for start, end in intervals for p in range(start, end)]
    if not selected:
        return base_cache
    _register()
    base = base_model(model)
    device = ids.device
    length = ids.shape[1]
    positions = torch.tensor(selected, dtype=torch.long, device=device)
    mask = (torch.arange(length, device=device)[None, :] <= positions[:, None])[None, None]
    output = clone_cache(base_cache)
    cache = Cache(layers=[_IndexCopyLayer(*layer_kv(output, i), positions) for i in range(len(output.layers))])
    view = _view_with_attention(base, _NAME)
    extra = {}
    if record is not None:
        record.update(inputs={}, attention={}, tables=None)
        for i, layer in enumerate(view.layers):
            layer.forward = _recording_forward(layer.forward, i, record)
        extra["oracle_record"] = record
    view(input_ids=ids.index_select(1, positions), position_ids=positions[None], past_key_values=cache,
         use_cache=True, oracle_packed_mask=mask, **extra)
    return output


@torch.no_grad()
def reference_refresh_stage(model, old_cache, old_ids, new_ids, intervals, record=None):
    """Shift cache (rotate) + packed SDPA refresh: the stage the bench times.
    With ``record``, also ``record["shifted"]``: the shifted cache the refresh
    started from (see packed_sdpa_repair for the per-layer records)."""
    shifted, _ = build_halo_cache(model, old_cache, old_ids, new_ids, 0)
    if record is not None:
        record["shifted"] = shifted
    return packed_sdpa_repair(model, shifted, new_ids, intervals, record)
