"""CPU checks of the readout's dropout definition and its oracle.

The HIP kernels drop attention weight s of row t of head h in batch b when a hash of
(seed, b, h, t, s) falls below round(p * 2^32) (include/wayfinder_hip.h,
wf_sparse_readout_fwd_dropout). Pinned here:
  * the C oracle's mask against a pure-Python evaluation of the header's definition
    (integer arithmetic, no shared code);
  * the mask's statistics: keep rate 1 - p, no correlation between neighbouring slots,
    rows or seeds;
  * the C dropout readout against the reference's formula in float64 torch,
    attn = dropout(softmax(scale q.k)) with the same mask (routing_attention/models/
    attention.py:35-55), and against the plain readout at p = 0;
  * the float64 autograd oracle with a mask against finite differences.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import native
from oracle.readout_grad import grads_autograd
from tests.helpers import rel_err

M32 = 0xFFFFFFFF


def _mix32(x: int) -> int:
    x ^= x >> 16
    x = (x * 0x7FEB352D) & M32
    x ^= x >> 15
    x = (x * 0x846CA68B) & M32
    x ^= x >> 16
    return x


def _keep(seed: int, r: int, s: int, p: float) -> bool:
    pf = float(torch.tensor(p, dtype=torch.float32))          # the ABI passes p as float32
    thresh = min(int(math.floor(pf * 4294967296.0 + 0.5)), M32)
    key = _mix32(_mix32((r & M32) ^ (seed & M32)) ^ (r >> 32) ^ ((seed >> 32) & M32))
    return _mix32(key ^ s) >= thresh


def test_mixer_known_values():
    # the integer hash is a bijection with mix(0) = 0; spot values computed by hand-checked
    # integer arithmetic above
    assert _mix32(0) == 0
    assert len({_mix32(x) for x in range(4096)}) == 4096


@pytest.mark.parametrize("p,seed", [(0.1, 1), (0.25, 12345), (0.5, 2 ** 40 + 7), (0.9, 2 ** 63 - 5)])
def test_c_mask_equals_header_definition(p, seed):
    B, H, T, K = 2, 3, 37, 20
    m = native.dropout_mask(B, H, T, K, p, seed)
    g = torch.Generator().manual_seed(seed % 1000)
    picks = torch.randint(0, B * H * T * K, (600,), generator=g).tolist()
    for e in picks:
        r, s = divmod(e, K)
        b, rem = divmod(r, H * T)
        h, t = divmod(rem, T)
        assert bool(m[b, h, t, s]) == _keep(seed, r, s, p), (b, h, t, s)


@pytest.mark.parametrize("p", [0.05, 0.1, 0.3, 0.5, 0.8])
def test_mask_statistics(p):
    B, H, T, K = 2, 4, 256, 128
    n = B * H * T * K
    m = native.dropout_mask(B, H, T, K, p, seed=99).double()
    keep = m.mean().item()
    sd = math.sqrt(p * (1 - p) / n)
    assert abs(keep - (1 - p)) < 5 * sd
    # neighbouring slots and rows look independent: P(both kept) = (1 - p)^2
    q2 = (1 - p) ** 2
    sd2 = math.sqrt(q2 * (1 - q2) / n)
    assert abs((m[..., 1:] * m[..., :-1]).mean().item() - q2) < 6 * sd2
    assert abs((m[:, :, 1:] * m[:, :, :-1]).mean().item() - q2) < 6 * sd2
    other = native.dropout_mask(B, H, T, K, p, seed=100).double()
    assert abs((m * other).mean().item() - q2) < 6 * sd2


def test_mask_deterministic_and_p_zero_keeps_everything():
    a = native.dropout_mask(1, 2, 30, 16, 0.3, 7)
    assert torch.equal(a, native.dropout_mask(1, 2, 30, 16, 0.3, 7))
    assert native.dropout_mask(1, 2, 30, 16, 0.0, 7).all()


def _inputs(B, H, T, D, K, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, T, D, generator=g) for _ in range(3))
    idx = torch.randint(0, T, (B, T, K), generator=g, dtype=torch.int32)
    return q, k, v, idx


@pytest.mark.parametrize("mask_pads", [False, True])
def test_c_dropout_readout_equals_reference_formula(mask_pads):
    B, H, T, D, K, p, seed = 2, 3, 40, 16, 12, 0.3, 4242
    q, k, v, idx = _inputs(B, H, T, D, K, seed=5)
    scale = D ** -0.5
    out = native.sparse_readout_dropout(q, k, v, idx, scale, p, seed, flags=int(mask_pads))
    keep = native.dropout_mask(B, H, T, K, p, seed)
    c = float(torch.tensor(1.0, dtype=torch.float32) / (1.0 - torch.tensor(p, dtype=torch.float32)))
    ref, *_ = grads_autograd(q, k, v, idx, scale, torch.zeros(B, H, T, D), mask_pads=mask_pads,
                             keep=keep, drop_scale=c)
    assert rel_err(out, ref) < 1e-12
    # p = 0 is the plain readout
    assert torch.equal(native.sparse_readout_dropout(q, k, v, idx, scale, 0.0, seed),
                       native.sparse_readout(q, k, v, idx, scale))


def test_masked_autograd_oracle_against_finite_differences():
    B, H, T, D, K = 1, 2, 9, 4, 5
    q, k, v, idx = _inputs(B, H, T, D, K, seed=11)
    keep = native.dropout_mask(B, H, T, K, 0.4, 77)
    scale = 0.5

    def f(q_, k_, v_):
        bi = torch.arange(B).view(B, 1, 1, 1)
        hi = torch.arange(H).view(1, H, 1, 1)
        ii = idx.long().unsqueeze(1)
        att = torch.softmax((q_.unsqueeze(3) * k_[bi, hi, ii, :]).sum(-1) * scale, dim=-1)
        att = att * keep.double() / 0.6
        return (att.unsqueeze(-1) * v_[bi, hi, ii, :]).sum(3)

    args = tuple(x.double().requires_grad_(True) for x in (q, k, v))
    assert torch.autograd.gradcheck(f, args)
    dout = torch.randn(B, H, T, D, dtype=torch.float64)
    _, dq, dk, dv = grads_autograd(q, k, v, idx, scale, dout, keep=keep, drop_scale=1 / 0.6)
    out = f(*args)
    out.backward(dout)
    for got, ref in ((dq, args[0].grad), (dk, args[1].grad), (dv, args[2].grad)):
        assert rel_err(got, ref) < 1e-12
