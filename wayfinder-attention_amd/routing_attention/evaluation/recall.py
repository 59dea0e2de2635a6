"""Recall@K of address / routing retrieval against attention (the reference's
routing_attention/evaluation/recall.py:110-141, ``compute_recall_at_k``: same name,
arguments and result keys).

The reference ranks every query's keys with a dense (B, T, T) similarity and
``torch.topk`` over it. Here, on a ROCm device, the predicted neighbours come from the HIP
streaming causal top-K run on the (query, key) vectors themselves, so no (B, T, T)
similarity is formed; only the ground-truth attention the caller passes in is (B, T, T).
Host tensors, a given ``similarity``, non-causal evaluation and vectors wider than the
kernel's address limit take a dense ranking with torch ops where the tensors live.

Metric (reference recall.py:89-107): per query, recall = |true ∩ pred| / k and precision =
|pred ∩ true| / k (each entry counted on its own side, so a duplicated index counts once
per occurrence), averaged over the queries whose causal attention row has any mass.

Semantics: predicted sets equal the reference's for every row t >= k_eff - 1 (exact fp32
scores, ties to the lower index). On rows t < k_eff - 1 the reference's dense top-K returns
whichever -inf (future) columns torch picks, this build the causal_topk pad indices: those
rows' hits are "parity unpinned".
"""

from __future__ import annotations

import torch
import torch.nn as nn

from routing_attention.kernels._common import has_hip
from routing_attention.kernels.causal_topk import MAX_ADDRESS_DIM, causal_topk


def _lower_triangle(T: int, device: torch.device) -> torch.Tensor:
    """(T, T) boolean mask of the causal pairs j <= t."""
    r = torch.arange(T, device=device)
    return r.view(T, 1) >= r.view(1, T)


def _membership_count(needles: torch.Tensor, haystack: torch.Tensor) -> torch.Tensor:
    """For (..., k) index sets: how many entries of ``needles`` occur in the same row of
    ``haystack`` (binary search in the sorted haystack)."""
    hay = haystack.sort(dim=-1).values.contiguous()
    pos = torch.searchsorted(hay, needles.contiguous()).clamp_(max=hay.shape[-1] - 1)
    return (hay.gather(-1, pos) == needles).sum(dim=-1)


def _recall_summary(true_idx: torch.Tensor, pred_idx: torch.Tensor, row_mass: torch.Tensor,
                    k_eff: int) -> dict[str, float]:
    """Mean recall / precision over the queries with positive attention mass."""
    true_idx, pred_idx = true_idx.long(), pred_idx.long()
    keep = row_mass > 0
    rec = _membership_count(true_idx, pred_idx).float()[keep] / k_eff
    prec = _membership_count(pred_idx, true_idx).float()[keep] / k_eff
    n = int(rec.numel())
    return {
        f"recall@{k_eff}": rec.mean().item() if n else 0.0,
        f"precision@{k_eff}": prec.mean().item() if n else 0.0,
        "num_queries": n,
        "mean_rank_true_neighbors": 0.0,
    }


def _head_flat(v: torch.Tensor) -> torch.Tensor:
    """(B, T, H, R) per-head vectors -> (B, T, H*R). The reference's head-mean similarity
    (sum over heads / H) ranks keys in the same order as the concatenated dot product."""
    return v.flatten(2) if v.dim() == 4 else v


def _stream_ok(q: torch.Tensor, k: torch.Tensor) -> bool:
    """The HIP top-K applies: device tensors, equal shapes, address dim within the limit."""
    return (q.is_cuda and k.is_cuda and q.shape == k.shape
            and _head_flat(q).shape[-1] <= MAX_ADDRESS_DIM and has_hip())


def _dense_similarity(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    if q.dim() == 4:   # per head, averaged over heads
        return torch.matmul(_head_flat(q), _head_flat(k).transpose(-2, -1)) / max(q.shape[2], 1)
    return torch.matmul(q, k.transpose(-2, -1))


def _topk_of_similarity(sim: torch.Tensor, k_eff: int, causal: bool) -> torch.Tensor:
    if causal:
        sim = sim.masked_fill(~_lower_triangle(sim.shape[-1], sim.device), float("-inf"))
    return torch.topk(sim, k=k_eff, dim=-1).indices


def _predicted(q: torch.Tensor, k: torch.Tensor, k_eff: int, causal: bool) -> torch.Tensor:
    if causal and _stream_ok(q, k):
        return causal_topk(_head_flat(q), _head_flat(k), k_eff)
    return _topk_of_similarity(_dense_similarity(q, k), k_eff, causal)


def _targets(attention: torch.Tensor, k_eff: int, causal: bool):
    """(true top-k indices of the causal attention, per-row attention mass)."""
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    if causal:
        attention = attention * _lower_triangle(attention.shape[-1], attention.device)
    return torch.topk(attention, k=k_eff, dim=-1).indices, attention.sum(dim=-1)


@torch.inference_mode()
def compute_recall_at_k(routing: torch.Tensor, attention: torch.Tensor, k: int = 32,
                        causal: bool = True, similarity: torch.Tensor | None = None,
                        include_mean_rank: bool = False) -> dict[str, float]:
    """Recall@K of ``routing`` (symmetric, r_i . r_j; (B,T,R) or per head (B,T,H,R)) or of a
    given dense ``similarity`` against the top-k of ``attention`` (B,T,T)
    (reference recall.py:110-141)."""
    del include_mean_rank
    k_eff = min(k, attention.shape[-1])
    true_idx, mass = _targets(attention, k_eff, causal)
    if similarity is not None:
        pred = _topk_of_similarity(similarity, k_eff, causal)
    else:
        pred = _predicted(routing, routing, k_eff, causal)
    return _recall_summary(true_idx, pred, mass, k_eff)


@torch.inference_mode()
def compute_recall_from_vectors(query: torch.Tensor, key: torch.Tensor, attention: torch.Tensor,
                                k: int = 32) -> dict[str, float]:
    """Recall@K of asymmetric (query, key) retrieval vectors -- e.g. the learned addresses of
    LearnedAddressModule.forward_query_key -- ranked by query_t . key_j over j <= t, with no
    (B, T, T) similarity on the device path. Attention (B,T,T) or (B,H,T,T) (head mean).
    No reference counterpart: the reference builds retrieval_scores first
    (learned_address.py:53-56) and ranks it."""
    k_eff = min(k, attention.shape[-1])
    true_idx, mass = _targets(attention, k_eff, True)
    return _recall_summary(true_idx, _predicted(query, key, k_eff, True), mass, k_eff)


@torch.inference_mode()
def compute_recall_from_addresses(hidden: torch.Tensor, attention: torch.Tensor,
                                  address_module: nn.Module, k: int = 32) -> dict[str, float]:
    """Recall@K of a LearnedAddressModule (or any module with forward_query_key) on hidden
    states (B, T, d_model): its addresses through compute_recall_from_vectors."""
    q, kk = address_module.forward_query_key(hidden)
    return compute_recall_from_vectors(q, kk, attention, k=k)
