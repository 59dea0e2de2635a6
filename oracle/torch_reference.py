"""Op-by-op PyTorch restatement of the reference's own path (test/baseline infrastructure).

This is the CPU baseline bench.py times and an independent cross-check of the C oracle's
index sets. It follows the reference's op sequence on purpose (it is the thing being
measured), in code of its own:

* ``row_blocked_topk``  -- routing_attention/kernels/causal_topk.py:470-521 (shape checks,
  k_eff, dtype promotion via _common.py:14-31) -> :132-171 (_causal_topk_row_blocked:
  fp32 cast, row blocks from _pick_row_block :75-83, bmm against the causal key prefix,
  masked_fill of j > t with -inf :110-129, topk(sorted=False)) -> :37-57 (finalize pads).
* ``sparse_meat_reference`` -- routing_attention/kernels/fused_sparse.py:64-94 (gather k/v
  at shared indices to (B,H,T,K,D), scores * scale, softmax, mul-then-sum), in the input
  dtype.
* ``fused_sparse_attention`` -- fused_sparse.py:327-356.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _row_block(T: int) -> int:
    # causal_topk.py:75-83
    for lim, bm in ((16384, 4096), (8192, 2048), (2048, 1024)):
        if T >= lim:
            return bm
    return 512


def _promote(q: torch.Tensor, k: torch.Tensor):
    # _common.py:14-31 with dtype=None
    target = q.dtype if q.dtype in (torch.float16, torch.bfloat16) else torch.float32
    return q.to(target), k.to(target)


def _finalize(vals: torch.Tensor, idx: torch.Tensor, k_eff: int) -> torch.Tensor:
    # causal_topk.py:37-57
    T = vals.shape[1]
    ok = torch.isfinite(vals) & (vals > -1e30)
    t = torch.arange(T, device=vals.device).view(1, T, 1)
    s = torch.arange(k_eff, device=vals.device).view(1, 1, k_eff)
    pad = (t + k_eff + s + 1) % T
    return torch.where(ok, idx.long(), pad).to(torch.int32)


@torch.no_grad()
def row_blocked_topk(query: torch.Tensor, key: torch.Tensor, top_k: int,
                     row_range: tuple[int, int] | None = None) -> torch.Tensor:
    """Reference retrieval, on the device of ``query`` (the CPU for the baseline; a GPU for
    the cross-check against torch's own GPU bmm / topk). ``row_range`` restricts the work
    to the row blocks that intersect [r0, r1); other rows are left -1."""
    if query.shape != key.shape:
        raise ValueError(f"query/key shape mismatch: {query.shape} vs {key.shape}")
    if query.dim() != 3:
        raise ValueError(f"expected (B,T,R), got {tuple(query.shape)}")
    B, T, _ = query.shape
    k_eff = min(top_k, T)
    if k_eff == 0:
        return torch.zeros(B, T, 0, dtype=torch.int32)
    q, k = _promote(query, key)
    q, k = q.float(), k.float()
    bm = _row_block(T)
    dev = q.device
    vals = torch.full((B, T, k_eff), float("-inf"), device=dev)
    idx = torch.full((B, T, k_eff), -1, dtype=torch.int32, device=dev)
    r0, r1 = row_range if row_range is not None else (0, T)
    for i0 in range(0, T, bm):
        i1 = min(i0 + bm, T)
        if i1 <= r0 or i0 >= r1:
            continue
        sc = torch.bmm(q[:, i0:i1], k[:, :i1].transpose(1, 2).contiguous())
        rows = torch.arange(i0, i1, device=dev).view(-1, 1)
        cols = torch.arange(i1, device=dev).view(1, -1)
        sc = sc.masked_fill((cols > rows).unsqueeze(0), float("-inf"))
        v, i = torch.topk(sc, k=k_eff, dim=-1, sorted=False)
        vals[:, i0:i1] = v
        idx[:, i0:i1] = i.to(torch.int32)
    out = _finalize(vals, idx, k_eff)
    if row_range is not None:
        keep = torch.zeros(T, dtype=torch.bool, device=dev)
        keep[r0:r1] = True
        out[:, ~keep] = -1
    return out


@torch.no_grad()
def sparse_meat_reference(q, k, v, indices, scale: float) -> torch.Tensor:
    """Reference readout (fused_sparse.py:64-94) in the input dtype."""
    B, H = k.shape[0], k.shape[1]
    bi = torch.arange(B).view(B, 1, 1, 1)
    hi = torch.arange(H).view(1, H, 1, 1)
    ii = indices.long().unsqueeze(1)
    k_sel = k[bi, hi, ii, :]
    v_sel = v[bi, hi, ii, :]
    sc = torch.matmul(q.unsqueeze(-2), k_sel.transpose(-2, -1)).squeeze(-2) * scale
    p = F.softmax(sc, dim=-1)
    return (p.unsqueeze(-1) * v_sel).sum(dim=-2)


@torch.no_grad()
def fused_sparse_attention(q_search, k_search, q, k, v, top_k: int, scale: float):
    idx = row_blocked_topk(q_search, k_search, top_k)
    return sparse_meat_reference(q, k, v, idx, scale), idx
