"""Skinny projection GEMMs of the packed refresh rows (libkvrepair kvr_linear_multi).

The packed executor recomputes only the selected rows (64 at a 64-token
budget), so every decoder projection is a [M <= 64, k] x [k, n] product that
streams the layer's weights once. A ProjectionPlan binds one projection's
weights (fixed for the life of a model) to the C entry point:

  * one weight:               y = x w^T                  (o_proj, down_proj)
  * concatenated weights:     y = x [w0; w1; w2]^T       (q/k/v into one output)
  * SiLU-gated pair:          y = act(x gate^T) * (x up^T)  (the MLP front half)
  * with a residual:          y = residual + x w^T          (down_proj + the layer's residual add)

Same results as torch.nn.functional.linear up to fp32 summation order (the
kernel accumulates in fp32 and rounds once); deterministic run to run. Plans
are pure host objects; the per-(device, stream) split-K workspace lives here.
"""

from __future__ import annotations

import ctypes
import threading
from typing import Sequence

import torch

from .. import _native

MAX_ROWS = 64
CONCAT = 0
SILU_GATE = 1
RESIDUAL = 2
_SUPPORTED = (torch.float16, torch.bfloat16)

_scratch_lock = threading.Lock()
_scratch: dict = {}


class _Scratch:
    """Split-K partials of one (device, stream): calls on one stream are
    ordered, so one buffer per stream serves every projection."""

    def __init__(self, device: torch.device):
        self.device = device
        self.workspace = torch.empty(0, dtype=torch.uint8, device=device)

    def reserve(self, workspace_bytes: int) -> torch.Tensor:
        if workspace_bytes > self.workspace.numel():
            self.workspace = torch.empty(workspace_bytes, dtype=torch.uint8, device=self.device)
        return self.workspace


def _scratch_for(device: torch.device, stream: int) -> _Scratch:
    key = (device.index, stream)
    entry = _scratch.get(key)
    if entry is None:
        with _scratch_lock:
            entry = _scratch.get(key)
            if entry is None:
                entry = _scratch[key] = _Scratch(device)
    return entry


def supported_weight(weight: torch.Tensor) -> bool:
    """A 2-D fp16/bf16 weight the kernel can stream: unit column stride, row
    stride a multiple of 8 elements, 16-byte aligned, k a multiple of 8."""
    return (isinstance(weight, torch.Tensor) and weight.ndim == 2 and weight.dtype in _SUPPORTED
            and weight.is_cuda and weight.stride(1) == 1 and weight.stride(0) % 8 == 0
            and weight.shape[1] % 8 == 0 and weight.data_ptr() % 16 == 0 and weight.shape[0] > 0)


class ProjectionPlan:
    """Bound ctypes arguments of one projection over fixed weights.

    Holds raw device pointers, not the tensors: the caller keeps the weights
    alive (the plans of the packed executor live no longer than one refresh
    or are revalidated against the weights' pointers, see ``matches``)."""

    def __init__(self, weights: Sequence[torch.Tensor], epilogue: int = CONCAT):
        weights = list(weights)
        if not 1 <= len(weights) <= 3 or not all(supported_weight(w) for w in weights):
            raise ValueError("projection plan needs 1-3 supported fp16/bf16 weights")
        k = int(weights[0].shape[1])
        if any(int(w.shape[1]) != k or w.dtype != weights[0].dtype or w.device != weights[0].device
               for w in weights):
            raise ValueError("projection plan weights must share k, dtype and device")
        if epilogue == SILU_GATE and (len(weights) != 2 or weights[0].shape != weights[1].shape):
            raise ValueError("SiLU-gated plan needs two weights of one shape (gate, up)")
        if epilogue not in (CONCAT, SILU_GATE):
            raise ValueError("unknown projection epilogue")
        self.epilogue = epilogue
        self.k = k
        self.dtype = weights[0].dtype
        self.device = weights[0].device
        self.rows = sum(int(w.shape[0]) for w in weights)
        self.n_out = int(weights[0].shape[0]) if epilogue == SILU_GATE else self.rows
        self.pointers = tuple(int(w.data_ptr()) for w in weights)
        self._w = (ctypes.c_void_p * len(weights))(*self.pointers)
        self._rows = (ctypes.c_int32 * len(weights))(*(int(w.shape[0]) for w in weights))
        self._ldw = _native.i64_array([int(w.stride(0)) for w in weights])
        self._count = len(weights)
        self._code = _native.DTYPE_CODES[self.dtype]
        self._workspace: dict[int, int] = {}

    def matches(self, weights: Sequence[torch.Tensor]) -> bool:
        return tuple(int(w.data_ptr()) for w in weights) == self.pointers

    def workspace_bytes(self, m: int) -> int:
        need = self._workspace.get(m)
        if need is None:
            need = int(_native.lib().kvr_linear_workspace_bytes(m, self.rows, self.k))
            _native.check(need, "kvr_linear_workspace_bytes")
            self._workspace[m] = need
        return need

    def __call__(self, x: torch.Tensor, stream: int | None = None, residual: torch.Tensor | None = None
                 ) -> torch.Tensor:
        """y[..., n_out] for x[..., k] (rows of x contiguous, at most MAX_ROWS of them);
        with ``residual`` (same shape as y, rows contiguous) y = residual + x w^T,
        rounded as the eager add rounds it."""
        if x.dtype != self.dtype or x.device != self.device or x.shape[-1] != self.k or x.stride(-1) != 1:
            raise RuntimeError("projection input geometry/dtype/device drifted")
        m = x.numel() // self.k
        if not 0 < m <= MAX_ROWS:
            raise RuntimeError(f"projection plans serve 1..{MAX_ROWS} rows, got {m}")
        rows2d = x.reshape(m, self.k)
        ldx = int(rows2d.stride(0))
        if stream is None:
            stream = torch.cuda.current_stream(self.device).cuda_stream
        need = self.workspace_bytes(m)
        workspace = _scratch_for(self.device, stream).reserve(need).data_ptr() if need else None
        y = torch.empty((*x.shape[:-1], self.n_out), dtype=self.dtype, device=self.device)
        epilogue, res, ldr = self.epilogue, None, 0
        if residual is not None:
            if self.epilogue != CONCAT or residual.shape != y.shape or residual.dtype != self.dtype \
                    or residual.device != self.device or residual.stride(-1) != 1:
                raise RuntimeError("projection residual geometry/dtype/device drifted")
            res2d = residual.reshape(m, self.n_out)
            epilogue, res, ldr = RESIDUAL, res2d.data_ptr(), int(res2d.stride(0))
        status = _native.lib().kvr_linear_multi(
            rows2d.data_ptr(), self._count, self._w, self._rows, self._ldw, y.data_ptr(), m, self.k, ldx,
            self.n_out, epilogue, res, ldr, workspace, need, self._code, ctypes.c_void_p(stream))
        _native.check(status, "kvr_linear_multi")
        return y


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """torch.nn.functional.linear(x, weight) (no bias) for at most MAX_ROWS rows."""
    return ProjectionPlan([weight])(x)


def linear_concat(x: torch.Tensor, weights: Sequence[torch.Tensor]) -> torch.Tensor:
    """torch.cat([F.linear(x, w) for w in weights], -1) in one launch (1-3 weights)."""
    return ProjectionPlan(weights, CONCAT)(x)


def silu_gate_linear(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(F.linear(x, gate)) * F.linear(x, up) with the eager ops' rounding, in one launch."""
    return ProjectionPlan([gate, up], SILU_GATE)(x)
