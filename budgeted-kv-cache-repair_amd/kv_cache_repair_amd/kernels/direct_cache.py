"""Direct interval repair: the sequential schedule writing fresh K/V in place.

Same public contract as the reference's experimental executor
(src/kv_cache_repair/kernels/direct_cache.py:147-226, ``direct_interval_repair``):
the interval recurrence of ``execution.sequential_repair`` (one native model
forward per maximal interval, each attending to the rows refreshed before it),
without the per-interval prefix views and concatenations. The output cache is
cloned once; during each interval's forward every layer is a cache adapter over
that output, which reports the interval's start as its length, writes the
forward's fresh K/V rows straight into rows [start, end) with
kvr_copy_kv_interval and hands attention the rows [0, end) (a strided view, or
a contiguous copy with ``attention_layout="contiguous"``, which is then the
exact tensor the sequential schedule builds).

The reference pins this prototype to transformers 4.57.6; this one is qualified
for the 5.15 classes the rest of the package serves (dense Llama and Qwen3,
eager or SDPA attention, full attention layers).
"""

from __future__ import annotations

import hashlib
import json
from typing import Any, Sequence

import torch
from transformers.cache_utils import Cache, DynamicLayer

from ..cache import OperatorShim, clone_cache, run_tokens_from_prefix
from .executor import _validate_cache, _validate_intervals, layer_kv
from .writeback import scatter_fresh_kv

# Writeback names the reference accepts ("torch" slice copies, its compiled
# "triton" scatter): both are served by the HIP interval copy here.
_WRITEBACKS = ("hip", "torch", "triton")


class _DirectIntervalLayer(DynamicLayer):
    """Owns no storage: one interval at a time, writes the native forward's
    fresh K/V into the matching layer of the owned output."""

    def __init__(self, key: torch.Tensor, value: torch.Tensor, contiguous: bool) -> None:
        super().__init__()
        self.keys, self.values = key, value
        self.dtype, self.device = key.dtype, key.device
        self.is_initialized = True
        self._contiguous = contiguous
        self._interval: tuple[int, int] | None = None
        self._updated = False

    def begin(self, start: int, end: int) -> None:
        if self._interval is not None:
            raise RuntimeError("previous interval transaction is still active")
        self._interval = (start, end)
        self._updated = False

    def finish(self) -> None:
        if self._interval is None or not self._updated:
            raise RuntimeError("native forward did not update every cache layer")
        self._interval = None

    def get_seq_length(self) -> int:
        # the forward numbers the interval's tokens from this length
        if self._interval is None:
            return int(self.keys.shape[-2])
        return self._interval[1] if self._updated else self._interval[0]

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        if self._interval is None:
            raise RuntimeError("mask requested outside an interval transaction")
        start, end = self._interval
        if int(query_length) != end - start:
            raise RuntimeError("native forward changed the interval position count")
        return end, 0

    def update(self, key_states, value_states, *args, **kwargs):
        if self._interval is None or self._updated:
            raise RuntimeError("expected exactly one update per layer and interval")
        start, end = self._interval
        expected = (*self.keys.shape[:2], end - start, self.keys.shape[-1])
        for source, target in ((key_states, self.keys), (value_states, self.values)):
            if source.shape != expected or source.dtype != target.dtype or source.device != target.device:
                raise RuntimeError("native cache update changed K/V shape, dtype, or device")
        scatter_fresh_kv(self.keys, self.values, key_states, value_states, start, end)
        self._updated = True
        key_rows, value_rows = self.keys[:, :, :end, :], self.values[:, :, :end, :]
        if self._contiguous:
            key_rows, value_rows = key_rows.contiguous(), value_rows.contiguous()
        return key_rows, value_rows


def _qualify_native_model(shim: Any, layer_count: int) -> None:
    """The exact native classes whose forward numbers positions from the cache
    length and asks the cache for its mask sizes (reference direct_cache.py:
    105-144, re-derived for transformers 5.15)."""
    from transformers import LlamaForCausalLM, LlamaModel, Qwen3ForCausalLM, Qwen3Model

    generator = shim.generator
    if getattr(generator, "training", True):
        raise ValueError("direct interval repair requires an eval-mode inference model")
    config = generator.config
    classes = {"llama": (LlamaForCausalLM, LlamaModel), "qwen3": (Qwen3ForCausalLM, Qwen3Model)}
    if config.model_type not in classes:
        raise ValueError("direct cache supports native Llama/Qwen3 models only")
    causal_type, base_type = classes[config.model_type]
    if type(generator) is not causal_type or type(OperatorShim._base_transformer(generator)) is not base_type:
        raise ValueError("direct cache requires the exact native model and base classes")
    if config._attn_implementation not in ("eager", "sdpa"):
        raise ValueError("direct cache supports eager or SDPA attention only")
    if config.num_hidden_layers != layer_count:
        raise ValueError("model and cache layer counts must match")
    if any(kind != "full_attention" for kind in getattr(config, "layer_types", []) or []):
        raise ValueError("direct cache does not support sliding/hybrid attention")
    if getattr(config, "use_sliding_window", False):
        raise ValueError("direct cache does not support sliding-window attention")


@torch.no_grad()
def direct_interval_repair(shim: Any, base_cache: Any, edited_ids_t: torch.Tensor,
                           intervals: Sequence[tuple[int, int]], *, writeback_backend: str = "torch",
                           attention_layout: str = "view") -> tuple[Any, dict[str, Any]]:
    """Interval forwards writing fresh K/V directly into one owned output.

    Returns an independently owned DynamicCache for a nonempty support and the
    borrowed base cache for an empty one; the base is never written, and a
    failed interval never exposes the partly written output. With
    ``attention_layout="contiguous"`` the result equals
    ``execution.sequential_repair`` bit for bit.
    """
    if writeback_backend not in _WRITEBACKS:
        raise ValueError("writeback_backend must be 'hip' (or the reference names 'torch' and 'triton', served by "
                         "the same HIP kernel)")
    if attention_layout not in ("view", "contiguous"):
        raise ValueError("attention_layout must be 'view' or 'contiguous'")
    if not isinstance(edited_ids_t, torch.Tensor) or edited_ids_t.ndim != 2 or edited_ids_t.shape[0] != 1:
        raise ValueError("edited_ids_t must be a single-batch rank-two tensor")
    if edited_ids_t.dtype not in (torch.int32, torch.int64):
        raise ValueError("edited_ids_t must contain int32 or int64 token IDs")
    length = int(edited_ids_t.shape[1])
    layer_count = _validate_cache(base_cache, length)
    validated = _validate_intervals(intervals, length)
    positions = [p for start, end in validated for p in range(start, end)]
    diagnostics = {
        "executor": "direct_interval_repair",
        "schedule": "reference_sequential_maximal_intervals",
        "writeback_backend": "hip",
        "writeback_validation": "owned_output_once_and_native_projection_per_update",
        "writeback_launch": "kvr_copy_kv_interval",
        "attention_layout": attention_layout,
        "interval_count": len(validated),
        "recomputed_tokens": len(positions),
        "rows_written_per_layer": len(positions),
        "layer_count": layer_count,
        "logical_length": length,
        "selection_positions_sha256": hashlib.sha256(
            json.dumps(positions, separators=(",", ":")).encode("utf-8")).hexdigest(),
        "conditioned_on_earlier_intervals": True,
        "base_cache_ownership": "borrowed_immutable",
        "output_cache_ownership": "independent" if validated else "borrowed_base",
        "attention_view_requires_numerical_qualification": attention_layout == "view",
    }
    if not validated:
        return base_cache, diagnostics
    _qualify_native_model(shim, layer_count)
    output = clone_cache(base_cache)
    contiguous = attention_layout == "contiguous"
    layers = [_DirectIntervalLayer(*layer_kv(output, i), contiguous) for i in range(layer_count)]
    adapter = Cache(layers=layers)
    for start, end in validated:
        for layer in layers:
            layer.begin(start, end)
        if run_tokens_from_prefix(shim, adapter, edited_ids_t[:, start:end], end) is not adapter:
            raise RuntimeError("native forward replaced the direct cache adapter")
        for layer in layers:
            layer.finish()
    return output, diagnostics
