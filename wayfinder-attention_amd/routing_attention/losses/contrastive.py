"""InfoNCE over causal address scores without a (B, T, T) similarity matrix (the reference's
routing_attention/losses/contrastive.py:163, batched_infonce_loss: same signature and value).

For query t: positives are the top_k keys of row t of the causally masked attention; the
loss is -(logsumexp over positives j <= t of s(t, j) - logsumexp over all j <= t of
s(t, j)), s = query . key / temperature (for per-head vectors (B, T, H, R): the head mean of
the per-head dot products), averaged over the queries that have a positive.

The reference forms the (B, T, T) similarity, a positive mask and a causal mask of the same
size. Here the rows are taken in blocks: positive scores are dot products with the
gathered positive keys (B, rows, top_k, R), and the causal log-sum-exp of a block is one
(B, rows, keys-so-far) product run under activation checkpointing, so autograd keeps only
the (B, T) results and recomputes each block's scores in the backward. Peak memory is one
block's scores instead of T x T.
"""

from __future__ import annotations

import torch
from torch.utils.checkpoint import checkpoint


def _flat(v: torch.Tensor) -> torch.Tensor:
    # (B, T, H, R) -> (B, T, H*R): the concatenated dot product is the sum over heads
    return v.flatten(2) if v.dim() == 4 else v


def _row_block(T: int) -> int:
    """Rows per block: about 64 Mi score elements per block at most."""
    return max(16, min(T, (1 << 26) // max(T, 1)))


def _causal_lse(q_blk: torch.Tensor, keys: torch.Tensor, i0: int, scale: float) -> torch.Tensor:
    """logsumexp_j<=t of scale * q_t . k_j for the rows t in [i0, i0 + rows)."""
    rows = q_blk.shape[1]
    i1 = i0 + rows
    s = torch.matmul(q_blk, keys[:, :i1].transpose(1, 2).contiguous()) * scale
    t = torch.arange(i0, i1, device=s.device).view(rows, 1)
    j = torch.arange(i1, device=s.device).view(1, i1)
    return torch.logsumexp(s.masked_fill((j > t).unsqueeze(0), float("-inf")), dim=-1)


def batched_infonce_loss(
    routing: torch.Tensor,
    attention: torch.Tensor,
    top_k: int = 32,
    temperature: float = 0.07,
    key_routing: torch.Tensor | None = None,
) -> torch.Tensor:
    """InfoNCE with the top_k attended keys of each query as positives and every causal key in
    the denominator (reference contrastive.py:163-204).

    Args:
        routing: (B, T, R) query vectors, or (B, T, H, R) per head.
        attention: (B, T, T) attention weights (row t over keys j).
        key_routing: key vectors of routing's shape (default: routing itself).
    """
    keys = routing if key_routing is None else key_routing
    heads = routing.shape[2] if routing.dim() == 4 else 1
    q, k = _flat(routing), _flat(keys)
    B, T = attention.shape[0], attention.shape[-1]
    k_eff = min(top_k, T)
    if k_eff <= 0 or T == 0:
        return torch.tensor(0.0, device=routing.device, requires_grad=True)
    scale = 1.0 / (temperature * heads)
    bm = _row_block(T)
    log_pos, log_all = [], []
    for i0 in range(0, T, bm):
        i1 = min(T, i0 + bm)
        t = torch.arange(i0, i1, device=attention.device).view(1, i1 - i0, 1)
        # positives: the top_k of the causally masked attention rows (future keys weigh 0)
        att = attention[:, i0:i1].masked_fill(torch.arange(T, device=attention.device).view(1, 1, T) > t, 0)
        pos = torch.topk(att, k=k_eff, dim=-1).indices                          # (B, rows, k)
        k_pos = torch.gather(k, 1, pos.reshape(B, -1, 1).expand(-1, -1, k.shape[-1]))
        s_pos = (q[:, i0:i1].unsqueeze(2) * k_pos.view(B, i1 - i0, k_eff, -1)).sum(-1) * scale
        # a positive in the future carries the causal mask's -inf, as in the reference
        log_pos.append(torch.logsumexp(s_pos.masked_fill(pos > t, float("-inf")), dim=-1))
        if q.requires_grad or k.requires_grad:
            log_all.append(checkpoint(_causal_lse, q[:, i0:i1], k, i0, scale, use_reentrant=False))
        else:
            log_all.append(_causal_lse(q[:, i0:i1], k, i0, scale))
    loss = -(torch.cat(log_pos, dim=1) - torch.cat(log_all, dim=1))            # (B, T)
    return loss.mean()
