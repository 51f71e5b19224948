"""Frozen-embedding query relevance on the GPU (libkvrepair kvr_query_relevance).

Same public contract as the reference's scorer (src/kv_cache_repair/scoring.py:
11-92): ``dense_query_relevance_scores(model=, edited_input_ids=,
query_token_ids=)`` returns one float per prompt token -- the largest cosine
between its embedding row and a query token's, plus 0.25 when the token id is
one of the query ids -- and the same metadata; ``query_text_token_ids``
tokenizes the query text. The reference's 1024-token chunks of eager ops and
host list comprehension become one kernel launch over every token; the
embedding must be a plain ``nn.Embedding`` on a ROCm device (no CPU path).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _native

_BOOST = 0.25


@torch.no_grad()
def dense_query_relevance_scores(*, model: Any, edited_input_ids: torch.Tensor,
                                 query_token_ids: list[int]) -> tuple[list[float], dict[str, Any]]:
    if not query_token_ids:
        raise ValueError("dense query scorer requires query tokens")
    embedding = model.generator.get_input_embeddings()
    weight = getattr(embedding, "weight", None)
    if type(embedding) is not torch.nn.Embedding or embedding.max_norm is not None or weight is None:
        raise ValueError("dense query scorer requires a plain nn.Embedding table")
    device = edited_input_ids.device
    if device.type != "cuda" or torch.version.hip is None:
        raise ValueError("dense query scorer runs on a ROCm GPU device")
    if weight.device != device:
        raise ValueError("embedding table and prompt ids must be on the same device")
    if weight.dtype not in _native.DTYPE_CODES or weight.ndim != 2 or weight.stride(1) != 1:
        raise ValueError("embedding table must be a row-major float32/float16/bfloat16 matrix")
    if edited_input_ids.ndim != 2 or edited_input_ids.shape[0] != 1 or \
            edited_input_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("edited_input_ids must be a [1, N] int32/int64 tensor")
    vocab = int(weight.shape[0])
    query = [int(value) for value in query_token_ids]
    if any(not 0 <= value < vocab for value in query):
        raise IndexError("index out of range in self")  # what the embedding lookup raises
    prompt = edited_input_ids[0]
    if prompt.stride(0) != 1:
        prompt = prompt.contiguous()
    n = int(prompt.shape[0])
    scores = torch.empty(n, dtype=torch.float32, device=device)
    query_dev = torch.tensor(query, dtype=torch.int64).pin_memory().to(device, non_blocking=True)
    status = _native.lib().kvr_query_relevance(
        weight.data_ptr(), vocab, int(weight.stride(0)), int(weight.shape[1]), prompt.data_ptr(),
        1 if prompt.dtype == torch.int32 else 0, n, query_dev.data_ptr(), len(query), _BOOST, scores.data_ptr(),
        _native.DTYPE_CODES[weight.dtype], _native.stream_handle(device))
    _native.check(status, "kvr_query_relevance")
    hidden_size = int(weight.shape[1])
    return [float(value) for value in scores.tolist()], {
        "query_token_ids": query,
        "query_token_count": len(query),
        "exact_token_boost": _BOOST,
        "embedding_dot_flops": 2 * n * len(query) * hidden_size,
        "embedding_dot_flops_scope": (
            "prompt-token by query-token embedding dot products only; "
            "excludes lookup, normalization, max reduction, and "
            "exact-token boost"
        ),
    }


def query_text_token_ids(tokenizer: Any, query_text: str) -> list[int]:
    """The query's token ids (no special tokens), repeats kept (reference scoring.py:75-89)."""
    token_ids = [int(value) for value in tokenizer(query_text, add_special_tokens=False)["input_ids"]]
    if not token_ids:
        raise ValueError("query text tokenization is empty")
    return token_ids
