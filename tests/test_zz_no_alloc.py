"""kvr_packed_causal_attention_noalloc (static scratch array, no allocation)
against kvr_packed_causal_attention (caller workspace), called through the C
ABI on the same inputs: two calls in a row, the second smaller, each
bit-identical to the workspace entry point; two calls enqueued back to back on
two streams without a host synchronisation (the library orders them on the
device, so they cannot overwrite each other's partials) each bit-identical to
the workspace entry point; a request beyond the scratch limit is refused before
anything runs."""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

pytestmark = pytest.mark.gpu


def _schedule(lib, native, positions, n_keys, hq, hkv, dim, dtype, chunk_keys=0):
    pos = native.i64_array(positions)
    args = (pos, len(positions), n_keys, hq, hkv, dim, native.DTYPE_CODES[dtype], chunk_keys)
    need = int(lib.kvr_attention_schedule(*args, None, 0))
    assert need > 0
    host = (ctypes.c_int32 * need)()
    assert lib.kvr_attention_schedule(*args, host, need) == need
    return host


def _case(device, seed, n_keys, positions, hq=32, hkv=8, dim=128, dtype=torch.bfloat16):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(1, len(positions), hq, dim, generator=gen).to(device=device, dtype=dtype).transpose(1, 2)
    k = torch.randn(1, hkv, n_keys, dim, generator=gen).to(device=device, dtype=dtype)
    v = torch.randn(1, hkv, n_keys, dim, generator=gen).to(device=device, dtype=dtype)
    return q, k, v


def _run(lib, native, q, k, v, positions, host, noalloc):
    device = q.device
    _, hq, n_sel, dim = q.shape
    _, hkv, n_keys, _ = k.shape
    out = torch.full((1, n_sel, hq, dim), float("nan"), dtype=q.dtype, device=device).transpose(1, 2)
    pos = torch.tensor(positions, dtype=torch.int64, device=device)
    sched = torch.frombuffer(host, dtype=torch.int32).to(device)
    strides = native.i64_array(native.strides3(q) + native.strides3(k) + native.strides3(v) + native.strides3(out))
    stream = native.stream_handle(device)
    common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), pos.data_ptr(), n_sel, hq, hkv, n_keys, dim,
              ctypes.c_float(dim ** -0.5), strides, sched.data_ptr(), len(host), host)
    if noalloc:
        status = lib.kvr_packed_causal_attention_noalloc(*common, native.DTYPE_CODES[q.dtype], stream)
    else:
        ws_bytes = int(lib.kvr_attention_workspace_bytes(host, len(host), hq, dim))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        status = lib.kvr_packed_causal_attention(*common, ws.data_ptr(), ws_bytes, native.DTYPE_CODES[q.dtype],
                                                 stream)
    assert status == 0, lib.kvr_status_string(status)
    torch.cuda.synchronize(device)
    return out


def test_noalloc_attention_matches_workspace_entry_point_on_two_calls(gpu_device):
    from kv_cache_repair_amd import _native

    lib = _native.lib()
    rng = random.Random(2)
    # first call: the bench geometry (16 intervals of 4 rows over 7680 keys, split-K partials in scratch);
    # second call: a smaller request (fewer rows and keys) on the same scratch array
    slots = sorted(rng.sample(range(5632 // 8), 16))
    big = [2048 + 8 * s + i for s in slots for i in range(4)]
    small = [300 + 3 * i for i in range(20)]
    for seed, (n_keys, positions) in enumerate(((7680, big), (1024, small))):
        print(f"noalloc attention case seed={seed} n_keys={n_keys} rows={len(positions)}", flush=True)
        q, k, v = _case(gpu_device, seed, n_keys, positions)
        host = _schedule(lib, _native, positions, n_keys, 32, 8, 128, q.dtype)
        assert lib.kvr_attention_workspace_bytes(host, len(host), 32, 128) > 0  # partials go through scratch
        want = _run(lib, _native, q, k, v, positions, host, noalloc=False)
        got = _run(lib, _native, q, k, v, positions, host, noalloc=True)
        assert torch.equal(got.contiguous().view(torch.int16), want.contiguous().view(torch.int16))
        assert not torch.isnan(got).any()


def test_noalloc_calls_on_two_streams_do_not_overlap(gpu_device):
    import bench
    from kv_cache_repair_amd import _native

    lib = _native.lib()
    rng = random.Random(3)
    slots = sorted(rng.sample(range(5632 // 8), 16))
    # a long call (the c4 bench layer: 1383 rows in 32 intervals over 31744 keys, 68 MB of partials)
    # and a short one (c3 geometry)
    c4 = bench.WORKLOADS["c4"]
    cases = [(c4.edited, c4.positions()), (7680, [2048 + 8 * s + i for s in slots for i in range(4)])]
    prepared = []
    for seed, (n_keys, positions) in enumerate(cases):
        print(f"noalloc two-stream case seed={seed} n_keys={n_keys} rows={len(positions)}", flush=True)
        q, k, v = _case(gpu_device, 10 + seed, n_keys, positions)
        host = _schedule(lib, _native, positions, n_keys, 32, 8, 128, q.dtype)
        need = lib.kvr_attention_workspace_bytes(host, len(host), 32, 128)
        assert 0 < need <= lib.kvr_attention_scratch_limit()
        want = _run(lib, _native, q, k, v, positions, host, noalloc=False)
        out = torch.full_like(want, float("nan"))
        pos = torch.tensor(positions, dtype=torch.int64, device=gpu_device)
        sched = torch.frombuffer(host, dtype=torch.int32).to(gpu_device)
        strides = _native.i64_array(_native.strides3(q) + _native.strides3(k) + _native.strides3(v)
                                    + _native.strides3(out))
        prepared.append((q, k, v, out, pos, sched, strides, host, want))
    torch.cuda.synchronize(gpu_device)
    streams = [torch.cuda.Stream(device=gpu_device) for _ in prepared]
    for (q, k, v, out, pos, sched, strides, host, _), stream in zip(prepared, streams):
        n_sel, n_keys = q.shape[2], k.shape[2]
        status = lib.kvr_packed_causal_attention_noalloc(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), pos.data_ptr(), n_sel, 32, 8, n_keys, 128,
            ctypes.c_float(128 ** -0.5), strides, sched.data_ptr(), len(host), host, _native.DTYPE_CODES[q.dtype],
            ctypes.c_void_p(stream.cuda_stream))
        assert status == 0, lib.kvr_status_string(status)
    torch.cuda.synchronize(gpu_device)
    for q, k, v, out, pos, sched, strides, host, want in prepared:
        assert torch.equal(out.contiguous().view(torch.int16), want.contiguous().view(torch.int16))


def test_noalloc_attention_refuses_requests_beyond_the_scratch_limit(gpu_device):
    from kv_cache_repair_amd import _native

    lib = _native.lib()
    limit = int(lib.kvr_attention_scratch_limit())
    assert limit == 128 << 20
    positions = list(range(8192, 8192 + 4096))
    host = _schedule(lib, _native, positions, 12288, 32, 8, 128, torch.bfloat16, chunk_keys=64)
    assert lib.kvr_attention_workspace_bytes(host, len(host), 32, 128) > limit
    q, k, v = _case(gpu_device, 7, 12288, positions)
    out = torch.zeros_like(q)
    pos = torch.tensor(positions, dtype=torch.int64, device=gpu_device)
    sched = torch.frombuffer(host, dtype=torch.int32).to(gpu_device)
    strides = _native.i64_array(_native.strides3(q) + _native.strides3(k) + _native.strides3(v)
                                + _native.strides3(out))
    status = lib.kvr_packed_causal_attention_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), pos.data_ptr(), len(positions), 32, 8, 12288, 128,
        ctypes.c_float(128 ** -0.5), strides, sched.data_ptr(), len(host), host, _native.DTYPE_CODES[q.dtype],
        _native.stream_handle(gpu_device))
    assert status == -10
    assert b"scratch" in lib.kvr_status_string(status)
    torch.cuda.synchronize(gpu_device)
    assert not out.any()  # nothing ran
