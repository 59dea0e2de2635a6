"""Recall@K on host tensors: no HIP top-K applies, so the functions rank a dense
similarity with torch ops on the CPU. Checked against the reference's formulas
(recall.py:89-141) restated here with broadcast comparisons."""

from __future__ import annotations

import torch

from routing_attention.evaluation import recall as R


def _attention(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, T, T, generator=g) * 3
    sc = sc.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    return torch.softmax(sc, dim=-1)


def _reference_recall(sim, attention, k):
    # reference recall.py:110-141 with :89-107 inlined
    T = attention.shape[-1]
    k_eff = min(k, T)
    tril = torch.tril(torch.ones(T, T))
    attn_masked = attention * tril.unsqueeze(0)
    sim = sim.masked_fill(tril.unsqueeze(0) == 0, float("-inf"))
    true = torch.topk(attn_masked, k_eff, dim=-1).indices
    pred = torch.topk(sim, k_eff, dim=-1).indices
    th = (true.unsqueeze(-1) == pred.unsqueeze(-2)).any(-1).float()
    ph = (pred.unsqueeze(-1) == true.unsqueeze(-2)).any(-1).float()
    valid = attn_masked.sum(-1) > 0
    return (th.sum(-1) / k_eff)[valid].mean().item(), (ph.sum(-1) / k_eff)[valid].mean().item(), int(valid.sum())


def test_recall_on_host_tensors_matches_reference_formula():
    g = torch.Generator().manual_seed(0)
    B, T, R_, k = 2, 40, 8, 4
    routing = torch.randn(B, T, R_, generator=g)
    attn = _attention(B, T, 1)
    got = R.compute_recall_at_k(routing, attn, k=k)
    rec, prec, n = _reference_recall(routing @ routing.transpose(1, 2), attn, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6
    assert got["num_queries"] == n
    # the advisor's case: uniform random attention, dim-8 routing, k=4
    out = R.compute_recall_at_k(torch.randn(1, 40, 8), torch.rand(1, 40, 40), k=4)
    assert 0.0 <= out["recall@4"] <= 1.0


def test_recall_from_vectors_and_similarity_on_host():
    g = torch.Generator().manual_seed(2)
    B, T, k = 1, 50, 6
    q, kk = torch.randn(B, T, 5, generator=g), torch.randn(B, T, 5, generator=g)
    attn = _attention(B, T, 3)
    got = R.compute_recall_from_vectors(q, kk, attn, k=k)
    rec, prec, _ = _reference_recall(q @ kk.transpose(1, 2), attn, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6
    sim = torch.randn(B, T, T, generator=g)
    got = R.compute_recall_at_k(None, attn, k=k, similarity=sim)
    rec, prec, _ = _reference_recall(sim, attn, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6


def test_recall_per_head_vectors_on_host():
    g = torch.Generator().manual_seed(4)
    B, T, H, k = 1, 30, 3, 5
    r = torch.randn(B, T, H, 4, generator=g)
    attn = _attention(B, T, 5)
    got = R.compute_recall_at_k(r, attn, k=k)
    sim = torch.einsum("bthq,bshq->bts", r, r) / H   # reference recall.py:125-126
    rec, prec, _ = _reference_recall(sim, attn, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6
