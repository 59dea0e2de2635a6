"""Pins of the gradient oracle (oracle/readout_grad.py) on the CPU: central finite
differences of the readout's forward, the closed-form row/key evaluators against autograd,
and the two size-independent identities the GPU tests use at full size."""

from __future__ import annotations

import pytest
import torch

from oracle import readout_grad as rg


def _case(B=1, H=2, T=40, D=8, K=6, seed=0, neg=True):
    g = torch.Generator().manual_seed(seed)
    q, k, v, dout = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(4))
    idx = torch.stack([torch.randint(0, t + 1, (B, K), generator=g) for t in range(T)], dim=1)
    idx[:, 5, 1] = idx[:, 5, 0]           # a duplicate slot
    if neg:
        idx[:, 7, 2] = -3                 # wraps to T-3 (torch advanced indexing)
        idx[:, 9, 0] = T + 5              # clamps to T-1
    return q, k, v, dout, idx.to(torch.int32)


def _f(q, k, v, idx, scale, dout, mask_pads):
    out, *_ = rg.grads_autograd(q, k, v, idx, scale, dout, mask_pads)
    return float((out * dout).sum())


@pytest.mark.parametrize("mask_pads", [False, True])
def test_autograd_oracle_matches_finite_differences(mask_pads):
    q, k, v, dout, idx = _case()
    scale = 0.35
    _, dq, dk, dv = rg.grads_autograd(q, k, v, idx, scale, dout, mask_pads)
    g = torch.Generator().manual_seed(1)
    eps = 1e-6
    for name, x, gx in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for _ in range(6):
            i = tuple(int(torch.randint(0, n, (1,), generator=g)) for n in x.shape)
            xp, xm = x.clone(), x.clone()
            xp[i] += eps
            xm[i] -= eps
            args = {"q": q, "k": k, "v": v}
            fp = _f(*[xp if n == name else args[n] for n in "qkv"], idx, scale, dout, mask_pads)
            fm = _f(*[xm if n == name else args[n] for n in "qkv"], idx, scale, dout, mask_pads)
            fd = (fp - fm) / (2 * eps)
            assert abs(fd - float(gx[i])) <= 1e-6 * max(1.0, abs(fd)), (name, i, fd, float(gx[i]))


@pytest.mark.parametrize("mask_pads", [False, True])
def test_closed_form_rows_and_keys_match_autograd(mask_pads):
    q, k, v, dout, idx = _case(B=2, H=2, T=30, D=8, K=8, seed=3)
    scale = 0.5
    _, dq, dk, dv = rg.grads_autograd(q, k, v, idx, scale, dout, mask_pads)
    rows = [0, 1, 5, 7, 9, 29]
    torch.testing.assert_close(rg.dq_rows(q, k, v, idx, scale, dout, rows, mask_pads), dq[:, :, rows],
                               rtol=1e-12, atol=1e-12)
    keys = [0, 3, 17, 27, 29]
    dk_s, dv_s = rg.dkdv_keys(q, k, v, idx, scale, dout, keys, mask_pads)
    torch.testing.assert_close(dk_s, dk[:, :, keys], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dv_s, dv[:, :, keys], rtol=1e-12, atol=1e-12)


def test_size_independent_identities():
    """<dq, q> = <dk, k> (scores are invariant under q -> c q, k -> k / c) and
    <dv, v> = <dout, out> (out is linear in v)."""
    q, k, v, dout, idx = _case(B=2, H=3, T=50, D=8, K=7, seed=5)
    out, dq, dk, dv = rg.grads_autograd(q, k, v, idx, 0.3, dout)
    assert abs(float((dq * q).sum() - (dk * k).sum())) < 1e-10
    assert abs(float((dv * v).sum() - (dout * out).sum())) < 1e-10
