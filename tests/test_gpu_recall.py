"""GPU checks of Recall@K on the streaming top-K (routing_attention/evaluation/recall.py)
against the reference's dense formulation (recall.py:89-141) restated here: predicted sets
from the C oracle, metrics recomputed with the reference's broadcast-compare formulas.

The ground-truth sets are torch.topk of the causal-masked attention on the GPU, as in the
reference; on rows t < k-1 they include zero-weight future columns chosen by torch's tie
handling, so the tests take the true sets from the same GPU computation."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.evaluation import recall as R
from routing_attention.models import LearnedAddressModule, RouterMLP

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _attention(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, T, T, generator=g) * 3
    sc = sc.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    return torch.softmax(sc, dim=-1)


def _ref_metrics(true_topk, pred_topk, attn_masked, k_eff):
    # reference recall.py:89-107 restated (broadcast comparison of the two index sets)
    th = (true_topk.unsqueeze(-1) == pred_topk.unsqueeze(-2)).any(-1).float()
    ph = (pred_topk.unsqueeze(-1) == true_topk.unsqueeze(-2)).any(-1).float()
    valid = attn_masked.sum(-1) > 0
    return (th.sum(-1) / k_eff)[valid].mean().item(), (ph.sum(-1) / k_eff)[valid].mean().item()


def _true_sets(attn, k, device):
    true, mass = R._targets(attn.to(device), k, True)
    am = attn * torch.tril(torch.ones(attn.shape[-1], attn.shape[-1]))
    return true.cpu(), am


def test_recall_from_addresses_matches_reference_formula(device):
    _say("[recall] learned addresses, B2 T512 k32")
    torch.manual_seed(0)
    B, T, k = 2, 512, 32
    mod = LearnedAddressModule(64, 16).to(device)
    hidden = torch.randn(B, T, 64, generator=torch.Generator().manual_seed(1)).to(device)
    attn = _attention(B, T, 2)
    got = R.compute_recall_from_addresses(hidden, attn.to(device), mod, k=k)
    with torch.no_grad():
        qa, ka = mod.forward_query_key(hidden)
    pred = native.causal_topk(qa.cpu(), ka.cpu(), k).long()
    true, am = _true_sets(attn, k, device)
    rec, prec = _ref_metrics(true, pred, am, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6
    assert got["num_queries"] == B * T
    # rows t >= k-1: the reference's dense top-K selects the same sets (near-ties aside)
    sim = qa.cpu().double() @ ka.cpu().double().transpose(1, 2)
    sim = sim.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    dense = torch.topk(sim, k, dim=-1).indices
    same = (dense.sort(-1).values == pred.sort(-1).values).all(-1)[:, k - 1:]
    assert same.float().mean() > 0.999


def test_recall_symmetric_routing(device):
    _say("[recall] symmetric routing vectors")
    B, T, k = 2, 300, 16
    r = torch.nn.functional.normalize(torch.randn(B, T, 24, generator=torch.Generator().manual_seed(3)), dim=-1)
    attn = _attention(B, T, 4)
    got = R.compute_recall_at_k(r.to(device), attn.to(device), k=k)
    pred = native.causal_topk(r, r, k).long()
    true, am = _true_sets(attn, k, device)
    rec, prec = _ref_metrics(true, pred, am, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6 and abs(got[f"precision@{k}"] - prec) < 1e-6


def test_recall_per_head_router_vectors(device):
    _say("[recall] per-head router vectors (flattened heads)")
    torch.manual_seed(5)
    B, T, k = 1, 256, 16
    router = RouterMLP(64, 8, similarity="asymmetric", n_heads=4, per_head_routing=True).to(device)
    hidden = torch.randn(B, T, 64, generator=torch.Generator().manual_seed(6)).to(device)
    attn = _attention(B, T, 7)
    with torch.no_grad():
        q, kk = router.forward_query_key(hidden)
        sim = router.retrieval_scores(hidden)
    got = R.compute_recall_from_vectors(q, kk, attn.to(device), k=k)
    # rows t >= k-1: the head-mean similarity and the flattened dot select the same sets
    # (up to rounding near-ties)
    sim = sim.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool, device=device), 1), float("-inf"))
    dense = torch.topk(sim, k, dim=-1).indices.sort(-1).values
    stream = R._predicted(q, kk, k, True).long().sort(-1).values
    assert (dense == stream).all(-1)[:, k - 1:].float().mean() > 0.99
    pred = native.causal_topk(q.reshape(B, T, -1).cpu(), kk.reshape(B, T, -1).cpu(), k).long()
    true, am = _true_sets(attn, k, device)
    rec, _ = _ref_metrics(true, pred, am, k)
    assert abs(got[f"recall@{k}"] - rec) < 1e-6
