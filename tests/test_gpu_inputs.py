"""GPU parity of kvr_refresh_inputs (embedding rows + rotary tables of the packed rows).

The reference obtains these from the model's own modules inside its packed
forward (src/kv_cache_repair/kernels/packed_cache.py:225-298): nn.Embedding and
the default-RoPE rotary embedding of transformers 5.15.0. Those modules are the
oracle here, run on the same GPU: the hidden rows must be the same bits, and the
cos/sin tables the same bits as the module's fp32 path rounded to the dtype.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

CONFIGS = [  # (rope theta, head_dim, model family)
    (5e5, 128, "llama"),
    (1e6, 128, "qwen3"),
    (1e4, 64, "llama"),
]


def rotary_module(theta, head_dim, family, device):
    if family == "qwen3":
        from transformers import Qwen3Config
        from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding as R

        cfg = Qwen3Config(hidden_size=head_dim * 8, num_attention_heads=8, num_key_value_heads=4, head_dim=head_dim,
                          rope_theta=theta)
    else:
        from transformers import LlamaConfig
        from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding as R

        cfg = LlamaConfig(hidden_size=head_dim * 8, num_attention_heads=8, num_key_value_heads=4, head_dim=head_dim,
                          rope_theta=theta)
    return R(cfg).to(device)


def call_inputs(ids, positions, weight, inv_freq, head_dim, scaling, hidden_out=None):
    from kv_cache_repair_amd import _native

    n = positions.numel()
    hidden_size = weight.shape[1]
    if hidden_out is None:
        hidden_out = torch.empty(n, hidden_size, dtype=weight.dtype, device=weight.device)
    cos = torch.empty(n, head_dim, dtype=weight.dtype, device=weight.device)
    sin = torch.empty_like(cos)
    status = _native.lib().kvr_refresh_inputs(
        ids.data_ptr(), 1 if ids.dtype == torch.int32 else 0, ids.numel(), positions.data_ptr(), n,
        weight.data_ptr(), weight.shape[0], weight.stride(0), hidden_size, hidden_out.data_ptr(),
        hidden_out.stride(0), inv_freq.data_ptr(), head_dim, ctypes.c_float(scaling), cos.data_ptr(), sin.data_ptr(),
        _native.DTYPE_CODES[weight.dtype], _native.stream_handle(weight.device))
    assert status == 0, status
    torch.cuda.synchronize()
    return hidden_out, cos, sin


def bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


@pytest.mark.parametrize("theta,head_dim,family", CONFIGS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("rows", ["c3_like", "sparse_far", "dense_c5"])
def test_inputs_match_the_model_modules_bit_for_bit(gpu_device, theta, head_dim, family, dtype, ids_dtype, rows):
    gen = torch.Generator().manual_seed(int(theta) % 9973 + head_dim)
    length = {"c3_like": 8192, "sparse_far": 131072, "dense_c5": 15104}[rows]
    if rows == "dense_c5":
        positions = torch.arange(length, dtype=torch.int64)
    else:
        positions = torch.randperm(length, generator=gen)[:64].sort().values
    vocab, hidden_size = 3000, 512
    weight = torch.randn(vocab, hidden_size, generator=gen).to(dtype).to(gpu_device)
    ids = torch.randint(0, vocab, (length,), generator=gen, dtype=torch.int64).to(ids_dtype).to(gpu_device)
    positions = positions.to(gpu_device)
    rotary = rotary_module(theta, head_dim, family, gpu_device)
    inv_freq = rotary.inv_freq.to(dtype=torch.float32).contiguous()
    hidden, cos, sin = call_inputs(ids, positions, weight, inv_freq, head_dim, float(rotary.attention_scaling))

    with torch.no_grad():
        want_hidden = torch.nn.functional.embedding(ids.index_select(0, positions).long(), weight)
        want_cos, want_sin = rotary(want_hidden[None], positions[None])
    assert torch.equal(bits(hidden), bits(want_hidden))
    assert torch.equal(bits(cos), bits(want_cos[0]))
    assert torch.equal(bits(sin), bits(want_sin[0]))


def test_inputs_scalar_path_strided_output_and_invalid_rows(gpu_device):
    """hidden_size 100 (rows not whole 16-byte vectors) into a strided output;
    an out-of-range token id and an out-of-range position give NaN rows only."""
    gen = torch.Generator().manual_seed(5)
    vocab, hidden_size, head_dim = 50, 100, 64
    weight = torch.randn(vocab, hidden_size + 3, generator=gen).to(torch.bfloat16).to(gpu_device)[:, :hidden_size]
    ids = torch.randint(0, vocab, (40,), generator=gen).to(gpu_device)
    ids[7] = vocab          # invalid token id at position 7
    ids[9] = -1             # and at position 9
    positions = torch.tensor([0, 7, 9, 12, 39, 40], dtype=torch.int64, device=gpu_device)  # 40: outside ids
    rotary = rotary_module(1e4, head_dim, "llama", gpu_device)
    inv_freq = rotary.inv_freq.float().contiguous()
    backing = torch.zeros(positions.numel(), hidden_size + 28, dtype=torch.bfloat16, device=gpu_device)
    hidden, cos, sin = call_inputs(ids, positions, weight, inv_freq, head_dim, 1.0,
                                   hidden_out=backing[:, 5:5 + hidden_size])
    valid = [0, 3, 4]
    want = torch.nn.functional.embedding(ids[positions[valid]], weight)
    assert torch.equal(bits(hidden[valid]), bits(want))
    for r in (1, 2, 5):
        assert torch.isnan(hidden[r].float()).all()
        assert torch.all(bits(hidden[r]) == 0x7FC0)
    assert torch.all(backing[:, :5] == 0) and torch.all(backing[:, 5 + hidden_size:] == 0)  # outside the view
    with torch.no_grad():
        want_cos, want_sin = rotary(hidden[None], positions[None])
    assert torch.equal(bits(cos), bits(want_cos[0])) and torch.equal(bits(sin), bits(want_sin[0]))
