"""kvr_upload_async: host ranges packed back to back into the library's pinned
staging and copied to the device on the caller's stream; more uploads in
flight than staging buffers; growth past the initial buffer size; refusal
under stream capture."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def upload(dst: torch.Tensor, parts: list[np.ndarray]) -> int:
    from kv_cache_repair_amd import _native

    count = len(parts)
    srcs = (ctypes.c_void_p * count)(*(p.ctypes.data if p.nbytes else None for p in parts))
    sizes = (ctypes.c_int64 * count)(*(p.nbytes for p in parts))
    return _native.lib().kvr_upload_async(dst.data_ptr(), srcs, sizes, count, _native.stream_handle(dst.device))


def test_upload_packs_the_ranges_in_order(gpu_device):
    rng = np.random.default_rng(1)
    parts = [rng.integers(0, 256, n, dtype=np.uint8) for n in (8, 0, 3, 100_000, 1, 70_000)]  # grows a buffer
    dst = torch.full((sum(p.nbytes for p in parts),), 7, dtype=torch.uint8, device=gpu_device)
    assert upload(dst, parts) == 0
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), np.concatenate(parts))


def test_more_uploads_in_flight_than_staging_buffers(gpu_device):
    """40 uploads behind a long kernel (the ring holds 8 buffers): each reuse
    waits for the buffer's earlier copy, so every destination gets its own
    bytes, and the host's ranges may be overwritten right after each call."""
    side = torch.cuda.Stream(device=gpu_device)
    side.wait_stream(torch.cuda.current_stream())
    host = np.empty(4096, dtype=np.int32)
    outs, want = [], []
    with torch.cuda.stream(side):
        torch.cuda._sleep(1_000_000)
        for i in range(40):
            host[:] = np.arange(4096, dtype=np.int32) * (i + 1)
            want.append(host.copy())
            out = torch.empty(host.nbytes, dtype=torch.uint8, device=gpu_device)
            assert upload(out, [host]) == 0
            outs.append(out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for out, expect in zip(outs, want):
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect)


def test_upload_is_refused_under_stream_capture(gpu_device):
    x = torch.zeros(16, device=gpu_device)
    dst = torch.zeros(64, dtype=torch.uint8, device=gpu_device)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=gpu_device)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        x.add_(1)  # warm the op outside capture
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph, stream=stream):
        x.add_(1)
        status = upload(dst, [np.ones(64, dtype=np.uint8)])
    assert status == -1
    torch.cuda.synchronize()
    assert int(dst.sum()) == 0
