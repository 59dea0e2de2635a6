"""CPU oracle of the sparse readout's gradients (indices fixed).

TEST INFRASTRUCTURE ONLY (imported by tests/, never by the product).

* ``grads_autograd``: float64 autograd of the reference's differentiable readout,
  routing_attention/models/attention.py:35-55 with _gather_kv_heads :58-69 (gather k/v at
  the shared indices, scores * scale, softmax, weighted sum of v), optionally with a given
  dropout mask on the weights. Pinned by
  ``torch.autograd.gradcheck`` (finite differences) in tests/test_oracle_grad.py.
* ``dq_rows`` / ``dkdv_keys``: the closed-form gradients evaluated for a subset of query
  rows or key rows in float64, for spot checks at sizes where the (B, H, T, K, D) gathers of
  the autograd version do not fit:
      p_s = softmax_s(scale q_t . k_{j_s}),  dp_s = dout_t . v_{j_s},  delta_t = sum_s p_s dp_s
      dq_t = scale sum_s p_s (dp_s - delta_t) k_{j_s}
      dk_j = scale sum_{(t, s): j_s = j} p_s (dp_s - delta_t) q_t,   dv_j = sum p_s dout_t
  They are cross-checked against ``grads_autograd`` on small inputs.
Index semantics follow the forward oracle: negative entries wrap by +T, the rest clamp to
[0, T-1]; with ``mask_pads`` slots s > t of rows t < K-1 carry no weight.
"""

from __future__ import annotations

import torch


def _norm_idx(indices: torch.Tensor, T: int) -> torch.Tensor:
    j = indices.long()
    j = torch.where(j < 0, j + T, j)
    return j.clamp(0, T - 1)


def _pad_mask(T: int, K: int) -> torch.Tensor:
    """(T, K) bool: True where slot s of row t carries no weight under mask_pads."""
    t = torch.arange(T).view(T, 1)
    s = torch.arange(K).view(1, K)
    return (t < K - 1) & (s > t)


def grads_autograd(q, k, v, indices, scale, dout, mask_pads=False, keep=None, drop_scale=1.0):
    """(out, dq, dk, dv) in float64 for (B, H, T, D) q/k/v/dout and (B, T, K) indices.
    ``keep`` (B, H, T, K) bool: dropout after the softmax (the reference's
    ``attn = dropout(softmax(...))`` with this mask), kept weights times ``drop_scale``."""
    q, k, v = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v))
    B, H, T, D = q.shape
    j = _norm_idx(indices.cpu(), T)
    K = j.shape[-1]
    bi = torch.arange(B).view(B, 1, 1, 1)
    hi = torch.arange(H).view(1, H, 1, 1)
    ii = j.unsqueeze(1)
    k_sel, v_sel = k[bi, hi, ii, :], v[bi, hi, ii, :]
    scores = (q.unsqueeze(3) * k_sel).sum(-1) * scale
    if mask_pads:
        scores = scores.masked_fill(_pad_mask(T, K).view(1, 1, T, K), float("-inf"))
    p = torch.softmax(scores, dim=-1)
    if keep is not None:
        p = p * keep.double() * float(drop_scale)
    out = (p.unsqueeze(-1) * v_sel).sum(dim=3)
    out.backward(dout.detach().cpu().double())
    return out.detach(), q.grad, k.grad, v.grad


def _row_terms(q, k, v, j, scale, dout, b, h, t, mask_pads):
    """p, ds (float64, length K) of one query row."""
    K = j.shape[-1]
    js = j[b, t]
    sc = (k[b, h, js] @ q[b, h, t]) * scale
    if mask_pads and t < K - 1:
        sc = sc.masked_fill(torch.arange(K) > t, float("-inf"))
    p = torch.softmax(sc, dim=0)
    dp = v[b, h, js] @ dout[b, h, t]
    delta = (p * dp).sum()
    return js, p, p * (dp - delta)


def dq_rows(q, k, v, indices, scale, dout, rows, mask_pads=False):
    """dq[b, h, t] for every (b, h) and t in ``rows``: float64 (B, H, len(rows), D)."""
    q, k, v, dout = (x.detach().cpu().double() for x in (q, k, v, dout))
    B, H, T, D = q.shape
    j = _norm_idx(indices.cpu(), T)
    out = torch.zeros(B, H, len(rows), D, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for r, t in enumerate(rows):
                js, _, ds = _row_terms(q, k, v, j, scale, dout, b, h, t, mask_pads)
                out[b, h, r] = scale * (ds @ k[b, h, js])
    return out


def dkdv_keys(q, k, v, indices, scale, dout, keys, mask_pads=False):
    """(dk, dv)[b, h, j] for every (b, h) and j in ``keys``: float64 (B, H, len(keys), D)
    each, summed over every (row, slot) that selected j."""
    q, k, v, dout = (x.detach().cpu().double() for x in (q, k, v, dout))
    B, H, T, D = q.shape
    j = _norm_idx(indices.cpu(), T)
    K = j.shape[-1]
    dk = torch.zeros(B, H, len(keys), D, dtype=torch.float64)
    dv = torch.zeros_like(dk)
    col = {int(key): r for r, key in enumerate(keys)}
    live = torch.zeros(T + 1, dtype=torch.bool)
    live[torch.tensor(list(col), dtype=torch.long)] = True
    for b in range(B):
        hit = live[j[b]]
        if mask_pads:
            hit &= ~_pad_mask(T, K)
        rows_b = hit.any(-1).nonzero().flatten().tolist()
        for h in range(H):
            for t in rows_b:
                js, p, ds = _row_terms(q, k, v, j, scale, dout, b, h, t, mask_pads)
                for s in hit[t].nonzero().flatten().tolist():
                    r = col[int(js[s])]
                    dk[b, h, r] += scale * ds[s] * q[b, h, t]
                    dv[b, h, r] += p[s] * dout[b, h, t]
    return dk, dv
