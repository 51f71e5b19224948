"""Public repair API over the MI355X packed refresh path.

Mirrors the reference public surface (src/kv_cache_repair/api.py):
``Selection``, ``RepairResult``, ``select_support`` and
``repair_after_deletion(..., executor="packed" | "sequential")``. Positional
correction (build_halo_cache), the packed refresh and the sequential
executor's writeback run on libkvrepair.

Support selection follows the reference (api.py:62-110): 0% selects nothing,
100% the whole suffix, and any budget in between the semantic-unit (SUR)
allocation over the GPU query-relevance scores (``semantic_units`` on the host,
``scoring.dense_query_relevance_scores`` on libkvrepair).
``repair_with_positions`` takes caller-selected positions instead.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Any, Sequence

import torch

from .alignment import token_alignment_arrays
from .cache import OperatorShim, build_halo_cache
from .execution import _refresh_intervals_, positions_to_intervals
from .scoring import dense_query_relevance_scores, query_text_token_ids
from .semantic_units import select_semantic_unit_support, semantic_unit_token_ranges
from .kernels.executor import layer_kv
from .kernels.packed_cache import _qualify, packed_refresh_owned_


@dataclass(frozen=True)
class Selection:
    """Selected absolute positions in the edited prompt, with half-open intervals."""

    positions: tuple[int, ...]
    intervals: tuple[tuple[int, int], ...]
    suffix_start: int
    suffix_tokens: int
    budget_tokens: int
    metadata: dict[str, Any]


@dataclass(frozen=True)
class RepairResult:
    """A repaired cache and the edited prompt it represents."""

    cache: Any
    edited_text: str
    input_ids: torch.Tensor
    selection: Selection
    metadata: dict[str, Any]


def _check_budget(budget_percent: float) -> float:
    if isinstance(budget_percent, bool):
        raise ValueError("budget_percent must be a number between 0 and 100")
    value = float(budget_percent)
    if not math.isfinite(value) or not 0.0 <= value <= 100.0:
        raise ValueError("budget_percent must be finite and between 0 and 100")
    return value


def _encode_host(model: Any, tokenizer: Any, text: str) -> torch.Tensor:
    """Token ids [1, tokens] (int64, host), checked against the embedding table:
    the refresh gathers embedding rows by these ids on the GPU, so an id outside
    the vocabulary is refused here, before any device work."""
    ids = tokenizer(text, add_special_tokens=False, return_tensors="pt")["input_ids"]
    if not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[0] != 1:
        raise ValueError("tokenizer must return input_ids with shape [1, tokens]")
    ids = ids.to(device="cpu", dtype=torch.long)
    vocab = int(model.get_input_embeddings().weight.shape[0])
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= vocab):
        raise ValueError(f"tokenizer returned token ids outside the model vocabulary [0, {vocab})")
    return ids


def _to_model_device(model: Any, ids: torch.Tensor) -> torch.Tensor:
    return ids.to(device=model.get_input_embeddings().weight.device)


def _selection(positions: Sequence[int], suffix_start: int, length: int, budget: int, metadata) -> Selection:
    positions = tuple(int(p) for p in positions)
    if len(positions) != budget or any(not suffix_start <= p < length for p in positions):
        raise RuntimeError("selected support violates the suffix budget")
    if any(b <= a for a, b in zip(positions, positions[1:])):
        raise ValueError("selected positions must be strictly increasing")
    return Selection(positions=positions, intervals=tuple(positions_to_intervals(list(positions))),
                     suffix_start=suffix_start, suffix_tokens=length - suffix_start, budget_tokens=budget,
                     metadata=metadata)


def _budget_selection(model: Any, tokenizer: Any, text: str, query: str, ids: torch.Tensor, suffix_start: int,
                      budget_percent: float) -> Selection:
    """``ceil(budget_percent / 100 * suffix_tokens)`` suffix positions of the
    edited prompt ``text`` (host ids ``ids``), as the reference selects them
    (api.py:62-110): none, the whole suffix, or the semantic-unit allocation
    over the query-relevance scores of every prompt token."""
    if isinstance(suffix_start, bool) or not isinstance(suffix_start, int):
        raise ValueError("suffix_start must be an integer token position")
    length = int(ids.shape[1])
    if not 0 <= suffix_start <= length:
        raise ValueError("suffix_start must lie inside the edited prompt")
    suffix_tokens = length - suffix_start
    budget = min(suffix_tokens, math.ceil(suffix_tokens * budget_percent / 100.0))
    metadata: dict[str, Any] = {"budget_percent": budget_percent}
    if budget == 0:
        metadata["selection"] = "shift_only"
        return _selection((), suffix_start, length, 0, metadata)
    if budget == suffix_tokens:
        metadata["selection"] = "full_suffix"
        return _selection(range(suffix_start, length), suffix_start, length, budget, metadata)
    units = semantic_unit_token_ranges(tokenizer=tokenizer, text=text, expected_token_ids=ids[0].tolist(),
                                       suffix_start=suffix_start)
    scores, scoring = dense_query_relevance_scores(model=OperatorShim(model, tokenizer),
                                                   edited_input_ids=_to_model_device(model, ids),
                                                   query_token_ids=query_text_token_ids(tokenizer, query))
    positions, allocator = select_semantic_unit_support(units=units, token_scores=scores, budget_tokens=budget)
    metadata.update({"selection": "sur", "scoring": scoring, "allocator": allocator})
    return _selection(positions, suffix_start, length, budget, metadata)


@torch.no_grad()
def select_support(model: Any, tokenizer: Any, edited_text: str, query: str, *, suffix_start: int,
                   budget_percent: float = 5.0) -> Selection:
    """``ceil(budget_percent / 100 * suffix_tokens)`` positions (reference api.py:113-132).

    0% selects nothing and 100% the whole suffix; other budgets take the
    semantic-unit allocation, whose scores need only the frozen input
    embeddings (one scorer launch, no transformer forward).
    """
    budget_percent = _check_budget(budget_percent)
    ids = _encode_host(model, tokenizer, edited_text)
    return _budget_selection(model, tokenizer, edited_text, query, ids, suffix_start, budget_percent)


def _check_model(model: Any) -> None:
    """Model contract of the reference (api.py:135-166) for transformers 5.15."""
    from transformers import LlamaForCausalLM, LlamaModel, Qwen3ForCausalLM, Qwen3Model

    base = getattr(model, "base_model", None)
    if (type(model), type(base)) not in {(LlamaForCausalLM, LlamaModel), (Qwen3ForCausalLM, Qwen3Model)}:
        raise ValueError("repair_after_deletion supports native dense Llama and Qwen3 models")
    if any(module.training for module in model.modules()):
        raise ValueError("call model.eval() before repairing its cache")
    config = model.config
    rope = getattr(config, "rope_parameters", None) or {}
    if rope.get("rope_type", "default") != "default" or getattr(base.rotary_emb, "rope_type", None) != "default":
        raise ValueError("repair requires default fixed RoPE")
    if (getattr(config, "use_sliding_window", False) or getattr(base, "has_sliding_layers", False)
            or any(kind != "full_attention" for kind in getattr(config, "layer_types", []) or [])):
        raise ValueError("repair requires full attention, not sliding or hybrid attention")
    if any(getattr(module, "_hf_hook", None) is not None for module in model.modules()):
        raise ValueError("repair does not support dispatch or offload hooks")
    if any("forward" in module.__dict__ for module in model.modules()):
        raise ValueError("repair does not support per-instance forward overrides")
    if getattr(model, "is_quantized", False):
        raise ValueError("repair does not support quantized models")
    # The device check comes last: every other rejection above is host-only and
    # names its cause whatever device the model is on.
    device = model.get_input_embeddings().weight.device
    if device.type != "cuda" or torch.version.hip is None or any(p.device != device for p in model.parameters()):
        raise ValueError("repair requires one ROCm GPU device holding every parameter")


def _check_span(original_text: str, delete_span) -> tuple[int, int]:
    if (not isinstance(delete_span, (tuple, list)) or len(delete_span) != 2
            or any(isinstance(v, bool) or not isinstance(v, int) for v in delete_span)):
        raise ValueError("delete_span must contain two integer character offsets")
    start, end = delete_span
    if not 0 <= start < end <= len(original_text):
        raise ValueError("delete_span must be a nonempty half-open span in original_text")
    return start, end


def _prepare(model, tokenizer, old_cache, original_text, start, end):
    """Model contract, both tokenizations (host) and the old cache's shape, in
    the reference's order (api.py:208-219); no device work."""
    _check_model(model)
    old_ids = _encode_host(model, tokenizer, original_text)
    old_length = int(old_ids.shape[1])
    layers = getattr(old_cache, "layers", None)
    if not old_length or layers is None or len(layers) != model.config.num_hidden_layers:
        raise ValueError("old_cache must contain every model layer for a nonempty prompt")
    device = model.get_input_embeddings().weight.device
    for i in range(len(layers)):
        key, value = layer_kv(old_cache, i)
        if key.ndim != 4 or key.shape != value.shape or key.shape[0] != 1 or key.shape[2] != old_length:
            raise ValueError("old_cache shape does not match the batch-one original prompt")
        if key.device != device or value.device != device:
            raise ValueError("cache and model must be on the same device")
    edited_text = original_text[:start] + original_text[end:]
    edited_ids = _encode_host(model, tokenizer, edited_text)
    return old_ids, edited_text, edited_ids


def _refresh(model, tokenizer, old_cache, old_ids, edited_ids, edited_text, selector, executor="packed"):
    """Select first (the suffix start comes from the host alignment, the same
    one build_halo_cache computes), so a selection error leaves no shifted cache
    behind; then shift and refresh the private shifted cache in place (packed:
    one pass over every selected row; sequential: the interval recurrence)."""
    alignment = token_alignment_arrays(old_ids[0].numpy(), edited_ids[0].numpy())
    selection = selector(int(edited_ids.shape[1]), int(alignment["new_suffix_start"]))
    shim = OperatorShim(model, tokenizer)
    edited_dev = _to_model_device(model, edited_ids)
    # host ids: the shift build reads them without waiting for the device
    shifted, alignment = build_halo_cache(shim, old_cache, old_ids, edited_ids, halo_tokens=0)
    if int(alignment["new_suffix_start"]) != selection.suffix_start:
        raise RuntimeError("host alignment and shift-cache alignment disagree")
    if executor == "packed":
        execution = packed_refresh_owned_(shim, shifted, edited_dev, list(selection.intervals))
    else:
        started = time.perf_counter()
        intervals = list(selection.intervals)
        _refresh_intervals_(shim, shifted, edited_dev, intervals)
        execution = {"executor": "sequential_interval_repair", "interval_count": len(intervals),
                     "recomputed_tokens": sum(e - s for s, e in intervals),
                     "seconds": time.perf_counter() - started, "conditioned_on_earlier_intervals": True}
    return RepairResult(cache=shifted, edited_text=edited_text, input_ids=edited_dev, selection=selection,
                        metadata={"alignment": alignment, "execution": execution, "executor": executor})


@torch.no_grad()
def repair_after_deletion(model: Any, tokenizer: Any, old_cache: Any, original_text: str, *,
                          delete_span: tuple[int, int], query: str, budget_percent: float = 5.0,
                          executor: str = "packed") -> RepairResult:
    """Delete a character span, correct positions, refresh selected suffix KV.

    Same contract as the reference (api.py:169-244): the input cache is never
    modified, boundary tokens whose tokenization changed are recomputed outside
    the suffix budget, and the returned cache is independently owned.
    ``executor="packed"`` refreshes every selected row in one pass on
    libkvrepair; ``"sequential"`` is the interval recurrence (one model forward
    per interval, each conditioned on the intervals before it, fresh rows
    written back by kvr_copy_kv_interval). The shifted cache built here is
    private, so either executor writes into it in place instead of cloning it
    again.
    """
    budget_percent = _check_budget(budget_percent)
    if executor not in ("packed", "sequential"):
        raise ValueError("executor must be 'packed' or 'sequential'")
    start, end = _check_span(original_text, delete_span)
    old_ids, edited_text, edited_ids = _prepare(model, tokenizer, old_cache, original_text, start, end)
    return _refresh(model, tokenizer, old_cache, old_ids, edited_ids, edited_text,
                    lambda length, suffix_start: _budget_selection(model, tokenizer, edited_text, query, edited_ids,
                                                                   suffix_start, budget_percent), executor)


@torch.no_grad()
def repair_with_positions(model: Any, tokenizer: Any, old_cache: Any, original_text: str, *,
                          delete_span: tuple[int, int], positions: Sequence[int]) -> RepairResult:
    """repair_after_deletion with caller-selected suffix positions (edited-prompt indices)."""
    start, end = _check_span(original_text, delete_span)
    old_ids, edited_text, edited_ids = _prepare(model, tokenizer, old_cache, original_text, start, end)
    chosen = tuple(int(p) for p in positions)

    def selector(length, suffix_start):
        return _selection(chosen, suffix_start, length, len(chosen), {"selection": "caller"})

    return _refresh(model, tokenizer, old_cache, old_ids, edited_ids, edited_text, selector)
