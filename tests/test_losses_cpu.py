"""The streaming InfoNCE (routing_attention/losses/contrastive.py) against the reference's
dense formulation (contrastive.py:163-204) restated here, value and gradients, on the CPU:
single and per-head vectors, asymmetric keys, rows whose positives reach into the future."""

from __future__ import annotations

import pytest
import torch

from routing_attention.losses import batched_infonce_loss
from routing_attention.losses import contrastive as C


def _reference(routing, attention, top_k, temperature, key_routing=None):
    # reference contrastive.py:148-204 restated: dense similarity, masks, logsumexps
    key = key_routing if key_routing is not None else routing
    if routing.dim() == 4:
        sim = torch.einsum("bthq,bshq->bts", routing, key) / max(routing.shape[2], 1)
    else:
        sim = torch.matmul(routing, key.transpose(-2, -1))
    sim = sim / temperature
    B, T, _ = attention.shape
    causal = torch.tril(torch.ones(T, T))
    attn_masked = attention * causal.unsqueeze(0)
    _, top_idx = torch.topk(attn_masked, k=min(top_k, T), dim=-1)
    positive = torch.zeros(B, T, T, dtype=torch.bool)
    positive.scatter_(2, top_idx, True)
    sim = sim.masked_fill(causal.unsqueeze(0) == 0, float("-inf"))
    log_pos = torch.logsumexp(sim.masked_fill(~positive, float("-inf")), dim=-1)
    log_all = torch.logsumexp(sim, dim=-1)
    valid = positive.any(dim=-1)
    return (-(log_pos - log_all))[valid].mean()


def _attention(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, T, T, generator=g) * 2
    return torch.softmax(sc.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf")), -1)


@pytest.mark.parametrize("shape,asym,k", [((2, 70, 8), False, 8), ((1, 90, 3, 4), True, 16), ((2, 40, 6), True, 5)])
def test_streaming_infonce_matches_dense_reference(shape, asym, k, monkeypatch):
    g = torch.Generator().manual_seed(sum(shape) + k)
    r = torch.randn(*shape, generator=g, dtype=torch.float64).requires_grad_(True)
    kr = torch.randn(*shape, generator=g, dtype=torch.float64).requires_grad_(True) if asym else None
    att = _attention(shape[0], shape[1], 7).double()
    monkeypatch.setattr(C, "_row_block", lambda T: 16)      # several blocks, ragged last one
    got = batched_infonce_loss(r, att, top_k=k, temperature=0.1, key_routing=kr)
    r2 = r.detach().clone().requires_grad_(True)
    kr2 = kr.detach().clone().requires_grad_(True) if asym else None
    want = _reference(r2, att, k, 0.1, kr2)
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)
    got.backward()
    want.backward()
    assert torch.allclose(r.grad, r2.grad, rtol=1e-9, atol=1e-12)
    if asym:
        assert torch.allclose(kr.grad, kr2.grad, rtol=1e-9, atol=1e-12)


def test_streaming_infonce_future_positives_and_k_over_T():
    """Rows t < k-1 take future (zero-attention) keys among their top-k: those carry the
    causal -inf in both formulations; k > T clamps to T."""
    g = torch.Generator().manual_seed(3)
    r = torch.randn(1, 12, 4, generator=g, dtype=torch.float64)
    att = _attention(1, 12, 4).double()
    for k in (6, 40):
        assert torch.allclose(batched_infonce_loss(r, att, top_k=k, temperature=0.5),
                              _reference(r, att, k, 0.5), rtol=1e-10)
