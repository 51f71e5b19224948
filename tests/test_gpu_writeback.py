"""GPU parity of the interval writeback (kvr_copy_kv_interval).

Mirrors the reference's tests/test_writeback.py with the HIP library in place
of Triton: bit-exact against torch's slice copy AND the C oracle over whole
backings (holes, permuted, batch/head holes, storage offsets), raw NaN payload
bits, and the validation contract (same ValueError classes and messages).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CODE = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16}


def _view(shape, dtype, layout, device):
    batch, heads, tokens, dim = shape
    if layout == "contiguous":
        backing = torch.randn(shape, device=device).to(dtype)
        return backing, backing
    if layout == "holes":
        backing = torch.randn((batch, heads, 2 * tokens + 3, 2 * dim + 5), device=device).to(dtype)
        return backing, backing[:, :, 1:1 + 2 * tokens:2, 2:2 + 2 * dim:2]
    if layout == "transposed":
        backing = torch.randn((batch, tokens, heads, dim), device=device).to(dtype)
        return backing, backing.permute(0, 2, 1, 3)
    if layout == "batch_head_holes":
        backing = torch.randn((2 * batch + 1, 2 * heads + 1, tokens + 2, dim + 4), device=device).to(dtype)
        return backing, backing[1:1 + 2 * batch:2, 1:1 + 2 * heads:2, 1:1 + tokens, 2:2 + dim]
    raise AssertionError(layout)


def host(t):
    t = t.detach().cpu()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,start,end", [((1, 8, 37, 128), 3, 4), ((2, 3, 71, 37), 5, 22),
                                             ((2, 5, 33, 7), 0, 33), ((1, 1, 9, 13), 0, 0),
                                             ((1, 8, 300, 128), 17, 289)])
@pytest.mark.parametrize("strided", [False, True])
def test_writeback_matches_slice_copy_oracle_and_preserves_storage(gpu_device, shape, start, end, dtype, strided):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    torch.manual_seed(701 + end)
    source_shape = (shape[0], shape[1], max(1, end), shape[3])
    layouts = ("holes", "transposed", "batch_head_holes", "holes") if strided else ("contiguous",) * 4
    pairs = [_view(s, dtype, layout, gpu_device)
             for s, layout in zip((shape, shape, source_shape, source_shape), layouts)]
    backings = [p[0] for p in pairs]
    tensors = [p[1] for p in pairs]
    snapshots = [b.clone() for b in backings]
    views = [b.as_strided(t.shape, t.stride(), t.storage_offset()) for b, t in zip(snapshots, tensors)]
    oracle_k = orc.copy_interval(host(views[0]), host(views[2]), start, start, end - start, CODE[dtype])
    oracle_v = orc.copy_interval(host(views[1]), host(views[3]), start, start, end - start, CODE[dtype])
    views[0][:, :, start:end, :].copy_(views[2][:, :, start:end, :])
    views[1][:, :, start:end, :].copy_(views[3][:, :, start:end, :])

    copy_kv_interval_(*tensors, start, end)
    torch.cuda.synchronize()
    # whole backings: unselected rows, holes, storage offsets and the sources are untouched
    for actual, expected in zip(backings, snapshots):
        assert torch.equal(actual.contiguous().view(torch.uint8), expected.contiguous().view(torch.uint8))
    assert np.array_equal(host(tensors[0]), oracle_k) and np.array_equal(host(tensors[1]), oracle_v)


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


@pytest.mark.parametrize("start,end", [(-1, 2), (2, 1), (0, 5), (True, 2), (0, 1.0)])
def test_invalid_interval_is_rejected(gpu_device, start, end):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    tensors = [torch.zeros((1, 2, 4, 8), device=gpu_device) for _ in range(4)]
    with pytest.raises(ValueError, match="interval"):
        copy_kv_interval_(*tensors, start, end)


@pytest.mark.parametrize("kind", ["source_alias", "output_alias", "dtype", "shape", "zero_stride", "overlap"])
def test_invalid_tensor_contract_is_rejected(gpu_device, kind):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    tensors = [torch.zeros((1, 2, 4, 8), device=gpu_device) for _ in range(4)]
    if kind == "source_alias":
        tensors[2] = tensors[0][:, :, :, :]
    elif kind == "output_alias":
        tensors[1] = tensors[0][:, :, :, :]
    elif kind == "dtype":
        tensors[2] = tensors[2].to(torch.float64)
    elif kind == "shape":
        tensors[2] = torch.zeros((1, 3, 4, 8), device=gpu_device)
    elif kind == "zero_stride":
        tensors[0] = torch.zeros((1, 1, 4, 8), device=gpu_device).expand(1, 2, 4, 8)
    elif kind == "overlap":
        tensors[0] = tensors[0].as_strided((1, 2, 4, 8), (64, 1, 1, 1))
    with pytest.raises(ValueError):
        copy_kv_interval_(*tensors, 0, 2)


@pytest.mark.parametrize("dtype,bits", [
    (torch.float16, [0, -32768, 31744, -1024, 32257, 1]),
    (torch.bfloat16, [0, -32768, 32640, -128, 32705, 1]),
])
def test_writeback_preserves_raw_bits_including_nan_payloads(gpu_device, dtype, bits):
    from kv_cache_repair_amd.kernels.writeback import copy_kv_interval_

    raw = torch.tensor(bits, dtype=torch.int16, device=gpu_device).reshape(1, 1, 2, 3)
    source_key = raw.view(dtype)
    source_value = source_key.clone()
    target_key = torch.zeros((1, 1, 4, 3), device=gpu_device, dtype=dtype)
    target_value = target_key.clone()
    copy_kv_interval_(target_key, target_value, source_key, source_value, 0, 2)
    torch.cuda.synchronize()
    for target in (target_key, target_value):
        assert torch.equal(target[:, :, :2, :].view(torch.int16), raw)
        assert torch.count_nonzero(target[:, :, 2:, :].view(torch.int16)) == 0
