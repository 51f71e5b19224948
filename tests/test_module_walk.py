"""The executor's module-tree walk (_kvr_walk.qualify_walk, C) against a Python
restatement of the same walk, on Llama and Qwen3 trees in the states the
qualification must notice: training mode, per-instance forwards, forward and
pre-forward hooks, dispatch hooks, empty module and parameter slots, tied
weights, an OrderedDict `_modules`, replaced modules and parameters."""

from __future__ import annotations

import collections

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

from kv_cache_repair_amd.kernels import packed_cache as pc


def subtree_dicts(root, skip):
    """__dict__ of `root` and every module under it, level by level through the
    `_modules` dicts, leaving out None entries and the subtree of `skip`."""
    found, level = [], [root.__dict__]
    while level:
        found += level
        level = [m.__dict__ for d in level for m in d["_modules"].values() if m is not None and m is not skip]
    return found


def python_walk(model, base):
    inner, outer = subtree_dicts(base, None), subtree_dicts(model, base)
    everything = inner + outer
    params = [p for d in everything for p in dict.values(d["_parameters"])]
    return (any(d["training"] for d in inner),
            any("forward" in d for d in inner),
            any(d.get("_hf_hook") is not None for d in everything),
            any(d["_forward_hooks"] or d["_forward_pre_hooks"] for d in inner),
            params,
            tuple(id(d) for d in everything),
            tuple(id(p) for p in params),
            tuple(torch.Tensor.data_ptr(p) for p in params if p is not None))


def c_walk(model, base):
    return pc._module_walk().qualify_walk(model, base, torch.Tensor.data_ptr)


def same(model):
    base = model.model
    expect, got = python_walk(model, base), c_walk(model, base)
    assert got[:4] == expect[:4]
    assert len(got[4]) == len(expect[4]) and all(a is b for a, b in zip(got[4], expect[4]))
    assert got[5:] == expect[5:]
    return got


def tiny(family):
    kw = dict(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=3, num_attention_heads=4,
              num_key_value_heads=2, head_dim=8)
    torch.manual_seed(0)
    if family == "llama":
        return LlamaForCausalLM(LlamaConfig(**kw)).eval()
    return Qwen3ForCausalLM(Qwen3Config(**kw)).eval()


@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_walk_matches_the_python_restatement(family):
    model = tiny(family)
    got = same(model)
    assert got[:4] == (False, False, False, False)
    # every module of the tree and every parameter slot, counted independently
    assert len(got[5]) == len(list(model.modules()))
    assert len(got[6]) == sum(len(m._parameters) for m in model.modules())


@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_walk_sees_each_disqualifying_state(family):
    model = tiny(family)
    base = model.model
    layer = base.layers[1]

    layer.mlp.train()
    assert same(model)[0] is True
    layer.mlp.eval()
    model.lm_head.train()  # outside the decoder: not an inner module
    assert same(model)[0] is False
    model.lm_head.eval()

    layer.self_attn.forward = lambda *args, **kwargs: None
    assert same(model)[1] is True
    del layer.self_attn.forward
    assert same(model)[1] is False

    model.lm_head._hf_hook = object()  # dispatch hooks count anywhere in the model
    assert same(model)[2] is True
    model.lm_head._hf_hook = None
    assert same(model)[2] is False

    handle = layer.mlp.down_proj.register_forward_hook(lambda *args: None)
    assert same(model)[3] is True
    handle.remove()
    handle = base.norm.register_forward_pre_hook(lambda *args: None)
    assert same(model)[3] is True
    handle.remove()
    handle = model.lm_head.register_forward_hook(lambda *args: None)  # outside the decoder
    assert same(model)[3] is False
    handle.remove()


def test_walk_follows_tree_edits():
    model = tiny("llama")
    base = model.model
    first = same(model)
    base.layers[0].mlp.up_proj = torch.nn.Linear(32, 48, bias=True)  # a replaced module, now with a bias
    second = same(model)
    assert second[5] != first[5] and second[6] != first[6] and len(second[7]) == len(first[7]) + 1
    proj = base.layers[2].self_attn.v_proj
    proj.weight.data = proj.weight.data.clone()  # same parameter, new storage
    third = same(model)
    assert third[6] == second[6] and third[7] != second[7]
    proj.register_parameter("extra", None)  # one more empty parameter slot
    fourth = same(model)
    assert len(fourth[6]) == len(third[6]) + 1 and len(fourth[7]) == len(third[7])
    base.layers[1]._modules["extra"] = None  # an empty module slot
    same(model)
    model.lm_head.weight = base.embed_tokens.weight  # tied weights: one tensor in two slots
    tied = same(model)
    assert tied[7].count(base.embed_tokens.weight.data_ptr()) == 2


def test_walk_reads_ordered_dict_module_maps_in_their_order():
    model = tiny("llama")
    layer = model.model.layers[0]
    layer._modules = collections.OrderedDict(layer._modules)
    layer._modules.move_to_end("self_attn")  # OrderedDict order differs from its dict storage order
    same(model)


def test_walk_raises_like_the_dict_lookups_it_replaces():
    model = tiny("llama")
    del model.model.layers[2].mlp.__dict__["training"]
    with pytest.raises(KeyError):
        python_walk(model, model.model)
    with pytest.raises(KeyError):
        c_walk(model, model.model)


@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_walk_with_the_layout_extensions_address_reader_matches(family):
    """The qualification passes the layout extension's data_ptr builtin as the
    walk's address reader: same walk result as with torch.Tensor.data_ptr."""
    from kv_cache_repair_amd.kernels.executor import tensor_layout

    model = tiny(family)
    base = model.model
    model.lm_head.weight = base.embed_tokens.weight  # one tensor in two slots
    with_method = pc._module_walk().qualify_walk(model, base, torch.Tensor.data_ptr)
    with_builtin = pc._module_walk().qualify_walk(model, base, tensor_layout().data_ptr)
    assert with_builtin[:4] == with_method[:4] and with_builtin[5:] == with_method[5:]
    assert all(a is b for a, b in zip(with_builtin[4], with_method[4]))
