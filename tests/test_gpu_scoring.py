"""GPU parity of the dense query relevance scorer (kvr_query_relevance).

Mirrors the reference's tests/test_scoring.py (its known-answer fixtures run on
the GPU here) and checks larger random inputs against the float64 oracle and a
torch float32 restatement of the reference's chunked eager ops
(scoring.py:11-72): tolerance 2e-6 absolute on cosines in [-1, 1] (fp32 sums
over up to 4096 products in a different order).
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _model(table: torch.Tensor):
    embedding = torch.nn.Embedding.from_pretrained(table, freeze=True)
    return SimpleNamespace(generator=SimpleNamespace(get_input_embeddings=lambda: embedding))


def _eager_f32(table: torch.Tensor, ids: torch.Tensor, query: list[int]) -> torch.Tensor:
    """The reference's chunked eager ops (scoring.py:27-62), float32 on the same device."""
    q = F.normalize(F.embedding(torch.tensor(query, device=table.device), table).float(), dim=-1)
    out = []
    for start in range(0, ids.shape[0], 1024):
        chunk = ids[start:start + 1024]
        sim = torch.matmul(F.normalize(F.embedding(chunk.long(), table).float(), dim=-1), q.t()).max(dim=1).values
        boost = torch.tensor([0.25 if int(t) in set(query) else 0.0 for t in chunk.tolist()], device=table.device)
        out.append(sim + boost)
    return torch.cat(out)


def test_exact_bonus_applies_only_to_identical_ids_kat(gpu_device):
    from kv_cache_repair_amd.scoring import dense_query_relevance_scores

    table = torch.tensor([[1.0, 0.0], [1.0, 0.0], [-1.0, 0.0], [0.0, 1.0]], device=gpu_device)
    scores, metadata = dense_query_relevance_scores(model=_model(table),
                                                    edited_input_ids=torch.tensor([[0, 1, 2, 3]], device=gpu_device),
                                                    query_token_ids=[1])
    assert scores == pytest.approx([1.0, 1.25, -1.0, 0.0])
    assert metadata["query_token_ids"] == [1]
    assert metadata["exact_token_boost"] == 0.25
    assert metadata["embedding_dot_flops"] == 16


def test_scores_are_preserved_across_the_reference_chunk_boundary_kat(gpu_device):
    from kv_cache_repair_amd.scoring import dense_query_relevance_scores

    table = torch.tensor([[1.0, 0.0], [1.0, 0.0], [-1.0, 0.0], [0.0, 1.0]], device=gpu_device)
    scores, _ = dense_query_relevance_scores(model=_model(table),
                                             edited_input_ids=torch.tensor([[2] * 1024 + [3]], device=gpu_device),
                                             query_token_ids=[1, 3])
    assert scores == pytest.approx([0.0] * 1024 + [1.25])


def test_rejects_empty_query_and_out_of_range_query_ids(gpu_device):
    from kv_cache_repair_amd.scoring import dense_query_relevance_scores

    model = _model(torch.randn(8, 4, device=gpu_device))
    ids = torch.tensor([[0]], device=gpu_device)
    with pytest.raises(ValueError, match="requires query tokens"):
        dense_query_relevance_scores(model=model, edited_input_ids=ids, query_token_ids=[])
    with pytest.raises(IndexError, match="index out of range"):
        dense_query_relevance_scores(model=model, edited_input_ids=ids, query_token_ids=[8])
    with pytest.raises(ValueError, match="ROCm GPU"):
        dense_query_relevance_scores(model=_model(torch.randn(8, 4)), edited_input_ids=torch.tensor([[0]]),
                                     query_token_ids=[1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
# token counts pick each MFMA launch shape (hidden axis over 1, 2, 4 or 8 waves): 40000 and 36000 -> 1,
# 20000 -> 2, 12000 -> 4, <= 10176 -> 8; up to 16 queries take one query tile per pass, more take four, more
# than 64 several passes
@pytest.mark.parametrize("hidden,n,n_query", [(4096, 20000, 20), (1024, 40000, 70), (256, 36000, 9),
                                             (512, 12000, 3), (256, 900, 100), (100, 3001, 5), (2048, 1025, 17),
                                             (64, 7, 1)])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_scores_match_the_oracle_and_the_eager_restatement(gpu_device, dtype, hidden, n, n_query, ids_dtype):
    from kv_cache_repair_amd.scoring import dense_query_relevance_scores

    gen = torch.Generator().manual_seed(hidden + n + n_query)
    vocab = 5000
    table = (torch.randn(vocab, hidden, generator=gen) * torch.rand(vocab, 1, generator=gen) * 3).to(dtype)
    ids = torch.randint(0, vocab, (n,), generator=gen)
    query = torch.randint(0, vocab, (n_query,), generator=gen).tolist()
    ids[:: max(1, n // 50)] = query[0]  # exact-id hits
    table_dev, ids_dev = table.to(gpu_device), ids.to(ids_dtype).to(gpu_device)
    scores, metadata = dense_query_relevance_scores(model=_model(table_dev), edited_input_ids=ids_dev[None],
                                                    query_token_ids=query)
    got = np.array(scores)
    want = orc.query_relevance_f64(table.float().numpy(), ids.numpy(), query)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    eager = _eager_f32(table_dev.float(), ids_dev.long(), query).cpu().numpy()
    np.testing.assert_allclose(got, eager, rtol=0, atol=2e-6)
    assert metadata["embedding_dot_flops"] == 2 * n * n_query * hidden


def test_out_of_range_token_ids_give_nan_scores_only_there(gpu_device):
    from kv_cache_repair_amd import _native

    table = torch.randn(16, 64, device=gpu_device).to(torch.bfloat16)
    ids = torch.tensor([0, 16, 3, -1, 15], device=gpu_device)
    query = torch.tensor([3, 5], device=gpu_device)
    scores = torch.full((5,), 7.0, device=gpu_device)
    status = _native.lib().kvr_query_relevance(table.data_ptr(), 16, 64, 64, ids.data_ptr(), 0, 5, query.data_ptr(),
                                               2, ctypes.c_float(0.25), scores.data_ptr(), 2,
                                               _native.stream_handle(gpu_device))
    assert status == 0
    torch.cuda.synchronize()
    got = scores.cpu()
    assert torch.isnan(got[[1, 3]]).all() and torch.isfinite(got[[0, 2, 4]]).all()
    want = orc.query_relevance_f64(table.float().cpu().numpy(), [0, 3, 15], [3, 5])
    np.testing.assert_allclose(got[[0, 2, 4]].numpy(), want, rtol=0, atol=2e-6)
