"""Recall@K of routing / address retrieval against attention (mirrors
routing_attention/evaluation/recall.py of the reference: same function names, arguments
and result keys).

The reference ranks every query's keys with a dense (B, T, T) similarity
(``router.retrieval_scores`` or ``routing @ routing^T``, recall.py:119-141, :155-175,
learned_address.py:53-56) and ``torch.topk`` over it. Here the predicted neighbours come
from the HIP streaming causal top-K on the (query, key) vectors themselves, so no (B, T, T)
similarity exists; only the ground-truth attention the caller passes in is (B, T, T).

Semantics: predicted sets equal the reference's for every row t >= k_eff - 1 (exact fp32
scores, ties to the lower index). On rows t < k_eff - 1 the reference's dense top-K returns
whichever -inf (future) columns torch picks, this build the causal_topk pad indices: those
rows' hits are "parity unpinned". A given ``similarity``, a non-causal evaluation, or vectors
wider than the kernel's 128 dims use the dense formulation of the reference (torch ops on
the tensors' device); host tensors on the streaming path raise, as every HIP entry does.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn

from routing_attention.kernels.causal_topk import causal_topk
from routing_attention.models.learned_address import PerLayerAddressBook
from routing_attention.models.router import PerLayerRouter

_MAX_STREAM_DIM = 128
_BIN_EDGES = [0, 1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 10000]   # reference recall.py:213
_CAUSAL_CACHE: dict[tuple[int, torch.device], torch.Tensor] = {}


def _causal_mask(seq_len: int, device: torch.device) -> torch.Tensor:
    key = (seq_len, device)
    if key not in _CAUSAL_CACHE:
        _CAUSAL_CACHE[key] = torch.tril(torch.ones(seq_len, seq_len, device=device))
    return _CAUSAL_CACHE[key]


def resolve_max_eval_tokens(seq_len: int, max_eval_tokens: int = 0, dry_run: bool = False) -> int:
    """How many token positions to score, 0 = auto (reference recall.py:25-41)."""
    if max_eval_tokens > 0:
        return min(max_eval_tokens, seq_len)
    if dry_run and seq_len <= 784:
        return seq_len
    if dry_run:
        return min(128, seq_len)
    for lim, n in ((4096, 256), (2048, 384), (1024, 512)):
        if seq_len > lim:
            return n
    return seq_len


def subsample_for_eval(hidden, attention, max_samples: int = 0):
    """Random subset of sequences (reference recall.py:44-53)."""
    if max_samples <= 0 or hidden.shape[0] <= max_samples:
        return hidden, attention
    idx = torch.randperm(hidden.shape[0], device=hidden.device)[:max_samples]
    return hidden[idx], attention[idx]


def subsample_tokens_for_eval(hidden, attention, max_tokens: int = 0):
    """Sorted random subset of positions, causal submatrix (reference recall.py:56-70)."""
    if max_tokens <= 0 or hidden.shape[1] <= max_tokens:
        return hidden, attention
    idx = torch.randperm(hidden.shape[1], device=hidden.device)[:max_tokens].sort().values
    hidden = hidden[:, idx]
    attention = attention[:, :, idx][:, :, :, idx] if attention.dim() == 4 else attention[:, idx][:, :, idx]
    return hidden, attention


def prepare_eval_tensors(hidden, attention, device, max_samples: int = 0, max_tokens: int = 0):
    """Subsample where the tensors are, then move the slice (reference recall.py:73-87)."""
    hidden, attention = subsample_for_eval(hidden, attention, max_samples)
    hidden, attention = subsample_tokens_for_eval(hidden, attention, max_tokens)
    nb = device.type == "cuda"
    return hidden.to(device, non_blocking=nb), attention.to(device, non_blocking=nb)


def _overall_recall_from_topk(true_topk, pred_topk, attn_masked, k_eff: int) -> dict[str, float]:
    """Recall / precision per query, averaged over queries with any attention mass
    (reference recall.py:90-107)."""
    true_hits = (true_topk.unsqueeze(-1) == pred_topk.unsqueeze(-2)).any(dim=-1).float()
    pred_hits = (pred_topk.unsqueeze(-1) == true_topk.unsqueeze(-2)).any(dim=-1).float()
    valid = attn_masked.sum(dim=-1) > 0
    recall = (true_hits.sum(dim=-1) / k_eff)[valid]
    precision = (pred_hits.sum(dim=-1) / k_eff)[valid]
    return {
        f"recall@{k_eff}": recall.mean().item() if recall.numel() else 0.0,
        f"precision@{k_eff}": precision.mean().item() if precision.numel() else 0.0,
        "num_queries": int(recall.numel()),
        "mean_rank_true_neighbors": 0.0,
    }


def _flat(v: torch.Tensor) -> torch.Tensor:
    """(B, T, H, R) per-head vectors -> (B, T, H*R): the head-mean similarity of the
    reference (sum over heads / H) ranks keys exactly as the concatenated dot product."""
    return v.reshape(v.shape[0], v.shape[1], -1) if v.dim() == 4 else v


def _streamable(q: torch.Tensor, k: torch.Tensor) -> bool:
    # host tensors are not streamable either: causal_topk raises for them (no CPU path)
    return _flat(q).shape[-1] <= _MAX_STREAM_DIM and q.shape == k.shape


def _dense_sim(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    if q.dim() == 4:
        return torch.matmul(q.permute(0, 2, 1, 3), k.permute(0, 2, 3, 1).contiguous()).sum(1) / max(q.shape[2], 1)
    return torch.matmul(q, k.transpose(-2, -1))


def _pred_topk(q, k, k_eff: int, causal: bool = True):
    """Predicted neighbours (B, T, k_eff): streaming causal top-K, or the reference's dense
    top-K where the kernel does not apply."""
    if causal and _streamable(q, k):
        return causal_topk(_flat(q), _flat(k), k_eff).long()
    sim = _dense_sim(q, k)
    if causal:
        sim = sim.masked_fill(_causal_mask(sim.shape[-1], sim.device).unsqueeze(0) == 0, float("-inf"))
    return torch.topk(sim, k=k_eff, dim=-1).indices


def _true_topk(attention, k_eff: int, causal: bool = True):
    T = attention.shape[-1]
    attn_masked = attention * _causal_mask(T, attention.device).unsqueeze(0) if causal else attention
    return torch.topk(attn_masked, k=k_eff, dim=-1).indices, attn_masked


@torch.inference_mode()
def compute_recall_at_k(routing, attention, k: int = 32, causal: bool = True, similarity=None,
                        include_mean_rank: bool = False) -> dict[str, float]:
    """Recall@K of ``routing`` (symmetric, r_i . r_j) or of a given dense ``similarity``
    against the top-k of ``attention`` (reference recall.py:110-141)."""
    del include_mean_rank
    T = attention.shape[-1]
    k_eff = min(k, T)
    true_topk, attn_masked = _true_topk(attention, k_eff, causal)
    if similarity is not None:
        sim = similarity
        if causal:
            sim = sim.masked_fill(_causal_mask(T, sim.device).unsqueeze(0) == 0, float("-inf"))
        pred_topk = torch.topk(sim, k=k_eff, dim=-1).indices
    else:
        pred_topk = _pred_topk(routing, routing, k_eff, causal)
    return _overall_recall_from_topk(true_topk, pred_topk, attn_masked, k_eff)


@torch.inference_mode()
def compute_recall_from_vectors(query, key, attention, k: int = 32) -> dict[str, float]:
    """Recall@K of asymmetric (query, key) retrieval vectors -- the learned addresses of
    LearnedAddressModule.forward_query_key -- with no (B, T, T) similarity. No reference
    counterpart: the reference goes through retrieval_scores (learned_address.py:53-56)."""
    T = attention.shape[-1]
    k_eff = min(k, T)
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    true_topk, attn_masked = _true_topk(attention, k_eff)
    return _overall_recall_from_topk(true_topk, _pred_topk(query, key, k_eff), attn_masked, k_eff)


def _router_vectors(router: nn.Module, hidden: torch.Tensor, layer_idx: int | None):
    if isinstance(router, (PerLayerRouter, PerLayerAddressBook)):
        assert layer_idx is not None
        return router.get_router(layer_idx).forward_query_key(hidden)
    if hasattr(router, "forward_query_key"):
        return router.forward_query_key(hidden)
    r = router(hidden)
    return r, r


@torch.inference_mode()
def compute_recall_from_router(hidden, attention, router: nn.Module, layer_idx: int | None = None,
                               k: int = 32, max_samples: int = 0, max_tokens: int = 0,
                               include_mean_rank: bool = False) -> dict[str, float]:
    """Recall@K of a router / address module on cached hidden states (reference
    recall.py:144-175), ranking with its (query, key) vectors on the streaming top-K."""
    del include_mean_rank
    device = next(router.parameters()).device
    hidden, attention = prepare_eval_tensors(hidden, attention, device, max_samples, max_tokens)
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    q, kv = _router_vectors(router, hidden, layer_idx)
    return compute_recall_from_vectors(q, kv, attention, k=k)


@torch.inference_mode()
def compute_recall_by_distance(routing, attention, k: int = 32, distance_buckets=None,
                               similarity=None, max_samples: int = 0, max_tokens: int = 0,
                               key_routing=None) -> dict[str, Any]:
    """Recall stratified by |i - j| of the true neighbours (reference recall.py:178-235).
    ``key_routing`` (this build's addition) gives asymmetric key vectors."""
    del distance_buckets
    device = routing.device
    routing, attention = prepare_eval_tensors(routing, attention, device, max_samples, max_tokens)
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    T = attention.shape[-1]
    k_eff = min(k, T)
    true_topk, attn_masked = _true_topk(attention, k_eff)
    if similarity is not None:
        sim = similarity.masked_fill(_causal_mask(T, similarity.device).unsqueeze(0) == 0, float("-inf"))
        pred_topk = torch.topk(sim, k=k_eff, dim=-1).indices
    else:
        pred_topk = _pred_topk(routing, routing if key_routing is None else key_routing, k_eff)
    query_pos = torch.arange(T, device=attention.device).view(1, T, 1)
    dist_true = (query_pos - true_topk).abs()
    in_pred = (true_topk.unsqueeze(-1) == pred_topk.unsqueeze(-2)).any(dim=-1)
    per_bin = []
    for lo, hi in zip(_BIN_EDGES[:-1], _BIN_EDGES[1:]):
        in_bin = (dist_true > lo) & (dist_true <= hi)
        hits = (in_bin & in_pred).sum().item()
        total = in_bin.sum().item()
        per_bin.append({"distance_min": lo, "distance_max": hi, "recall": hits / max(total, 1),
                        "hits": hits, "total": total})
    return {"buckets": {}, "per_bin": per_bin,
            "overall": _overall_recall_from_topk(true_topk, pred_topk, attn_masked, k_eff)}


@torch.inference_mode()
def compute_recall_by_distance_from_router(hidden, attention, router: nn.Module,
                                           layer_idx: int | None = None, k: int = 32,
                                           max_samples: int = 0, max_tokens: int = 0) -> dict[str, Any]:
    """Distance-stratified recall of a router on cached hidden states (reference
    recall.py:238-270)."""
    device = next(router.parameters()).device
    hidden, attention = prepare_eval_tensors(hidden, attention, device, max_samples, max_tokens)
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    q, kv = _router_vectors(router, hidden, layer_idx)
    return compute_recall_by_distance(q, attention, k=k, key_routing=kv)


@torch.inference_mode()
def compute_key_vector_recall_from_hidden(hidden, attention, attn_module: nn.Module,
                                          k: int = 32) -> dict[str, float]:
    """Recall@K of the head-mean Q/K projections of an attention module (reference
    recall.py:317-337: similarity q_mean . k_mean)."""
    if not hasattr(attn_module, "q_proj"):
        raise TypeError("attn_module must be DenseAttention with q_proj/k_proj")
    B, T, _ = hidden.shape
    H, hd = attn_module.n_heads, attn_module.head_dim
    q = attn_module.q_proj(hidden).view(B, T, H, hd).transpose(1, 2).mean(dim=1)
    kk = attn_module.k_proj(hidden).view(B, T, H, hd).transpose(1, 2).mean(dim=1)
    if attention.dim() == 4:
        attention = attention.mean(dim=1)
    return compute_recall_from_vectors(q, kk, attention, k=k)
