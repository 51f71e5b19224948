"""Strided [B, H, T, D] test views over flat random storages (test helper).

Every view is ``storage.as_strided(...)`` with explicit strides and offset, so
``storage_index`` can say which storage element each view element is, and a
test can compute the expected storage after a copy or scatter independently of
the kernel. The layouts are those the reference's tests exercise: dense,
sparse (every other row and dim, offset into a padded block), token-major
([B, T, H, D] storage seen as [B, H, T, D], HF's projection output), and padded
batch/head axes.
"""

from __future__ import annotations

import numpy as np
import torch

LAYOUTS = ("dense", "sparse", "token_major", "padded")


def strided_over_storage(shape, dtype, device, layout, generator=None, scale=1.0):
    """(flat storage, view of ``shape`` in ``layout``) with N(0, scale^2) storage."""
    b, h, t, d = shape
    if layout == "dense":
        strides, offset, numel = (h * t * d, t * d, d, 1), 0, b * h * t * d
    elif layout == "sparse":  # rows 1, 3, 5, ... and dims 2, 4, 6, ... of (2T+3) x (2D+5) blocks
        rows, cols = 2 * t + 3, 2 * d + 5
        strides, offset, numel = (h * rows * cols, rows * cols, 2 * cols, 2), cols + 2, b * h * rows * cols
    elif layout == "token_major":
        strides, offset, numel = (t * h * d, d, h * d, 1), 0, b * t * h * d
    elif layout == "padded":  # odd batch/head slots of (2B+1, 2H+1, T+2, D+4), one row and two dims in
        hh, rr, cc = 2 * h + 1, t + 2, d + 4
        strides = (2 * hh * rr * cc, 2 * rr * cc, cc, 1)
        offset, numel = hh * rr * cc + rr * cc + cc + 2, (2 * b + 1) * hh * rr * cc
    else:
        raise ValueError(layout)
    storage = (torch.randn(numel, device=device, generator=generator) * scale).to(dtype)
    return storage, storage.as_strided((b, h, t, d), strides, offset)


def storage_index(view):
    """Storage element index of every element of ``view`` (same shape, int64)."""
    count = view.untyped_storage().nbytes() // view.element_size()
    return torch.arange(count, device=view.device).as_strided(view.shape, view.stride(), view.storage_offset())


def host_bits(t):
    """Host copy: fp32 as float32, 16-bit dtypes as their uint16 bit patterns."""
    t = t.detach().cpu()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def same_bits(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


# fp16 / bf16 bit patterns: +0, -0, +inf, -inf, a NaN with payload, the smallest subnormal
PAYLOADS = {torch.float16: [0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E01, 0x0001],
            torch.bfloat16: [0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC1, 0x0001]}


def payload_rows(dtype, heads, rows, dim, device):
    """int16 tensor [1, heads, rows, dim] cycling through PAYLOADS[dtype]."""
    pattern = torch.tensor(PAYLOADS[dtype], dtype=torch.int32).to(torch.int16)
    n = heads * rows * dim
    return pattern.repeat((n + pattern.numel() - 1) // pattern.numel())[:n].reshape(1, heads, rows, dim).to(device)
