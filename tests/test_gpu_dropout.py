"""GPU parity of dropout in the HIP readout (the reference's non-fused training readout,
routing_attention/models/attention.py:35-55: attn = dropout(softmax(scale q.k)), out =
attn v). The kernels draw the keep mask from a hash of (seed, b, h, t, slot), so the CPU
oracle reproduces it exactly: forward outputs are compared with the C oracle's dropout
readout, gradients with float64 autograd of the reference formula under the oracle's mask,
on the aligned and the generic readout kernels, with and without pad masking. The module's
training forward is checked the same way for a seed fixed through torch.manual_seed."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from oracle.readout_grad import grads_autograd
from routing_attention.kernels.sparse_autograd import draw_dropout_seed, sparse_readout
from tests.helpers import addresses, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(B, H, T, D, K, dtype, seed, layout="bthd"):
    g = torch.Generator().manual_seed(seed)
    if layout == "bthd":
        q, k, v = (torch.randn(B, T, H, D, generator=g).to(dtype).transpose(1, 2) for _ in range(3))
    else:   # a strided head dim: the generic kernel
        q, k, v = (torch.randn(B, H, T, 2 * D, generator=g).to(dtype)[..., ::2] for _ in range(3))
    qa, ka = addresses(B, T, 32, seed=seed + 1)
    idx = native.causal_topk(qa, ka, K)
    return q, k, v, idx


def _c(p):
    return float(torch.tensor(1.0, dtype=torch.float32) / (1.0 - torch.tensor(p, dtype=torch.float32)))


@pytest.mark.parametrize("B,H,T,D,K,dtype,layout,p,mask_pads", [
    (1, 8, 1024, 64, 128, torch.bfloat16, "bthd", 0.1, False),    # aligned kernel, 16-byte index loads
    (2, 4, 700, 64, 100, torch.float32, "bthd", 0.3, False),      # K not a multiple of 4
    (1, 2, 500, 128, 256, torch.float16, "bhtd", 0.5, True),       # D = 128, pads masked
    (1, 3, 300, 32, 40, torch.float32, "strided", 0.2, False),     # generic kernel
    (2, 2, 200, 96, 64, torch.bfloat16, "bthd", 0.25, True),       # D = 96, padded lane layout
])
def test_dropout_forward_matches_oracle(device, B, H, T, D, K, dtype, layout, p, mask_pads):
    _say(f"[dropout] fwd B{B} H{H} T{T} D{D} K{K} {dtype} {layout} p={p} pads={mask_pads}")
    q, k, v, idx = _inputs(B, H, T, D, K, dtype, seed=T + D, layout=layout)
    seed = 0x1234_5678_9ABC_DEF0 + T
    scale = D ** -0.5
    out = sparse_readout(q.to(device), k.to(device), v.to(device), idx.to(device), scale,
                         mask_pads=mask_pads, dropout_p=p, seed=seed)
    ref = native.sparse_readout_dropout(q, k, v, idx, scale, p, seed, flags=int(mask_pads))
    assert rel_err(out.float(), ref) < TOL[dtype]
    # the mask really drops about p of the weights: the output differs from the plain readout
    plain = native.sparse_readout(q, k, v, idx, scale, flags=int(mask_pads))
    assert rel_err(ref, plain) > 0.05


@pytest.mark.parametrize("D,dtype,p,mask_pads", [
    (64, torch.float32, 0.1, False),
    (128, torch.float32, 0.4, True),
    (64, torch.bfloat16, 0.2, False),
])
def test_dropout_backward_matches_reference_autograd(device, D, dtype, p, mask_pads):
    _say(f"[dropout] bwd D{D} {dtype} p={p} pads={mask_pads}")
    B, H, T, K = 1, 2, 300, 48
    q, k, v, idx = _inputs(B, H, T, D, K, dtype, seed=D + 3)
    dout = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(9)).to(dtype)
    seed, scale = 987654321, D ** -0.5
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = sparse_readout(qd, kd, vd, idx.to(device), scale, mask_pads=mask_pads, dropout_p=p, seed=seed)
    out.backward(dout.to(device))
    keep = native.dropout_mask(B, H, T, K, p, seed)
    ro, rq, rk, rv = grads_autograd(q, k, v, idx, scale, dout, mask_pads=mask_pads, keep=keep,
                                    drop_scale=_c(p))
    tol = 1e-5 if dtype == torch.float32 else 3e-2
    assert rel_err(out.detach().float(), ro) < tol
    assert rel_err(qd.grad.float(), rq) < tol
    assert rel_err(kd.grad.float(), rk) < tol
    assert rel_err(vd.grad.float(), rv) < tol


def test_dropout_seed_semantics(device):
    _say("[dropout] same seed same output, other seed other output, p=0 plain")
    q, k, v, idx = _inputs(1, 4, 512, 64, 128, torch.bfloat16, seed=21)
    q, k, v, idx = (x.to(device) for x in (q, k, v, idx))
    a = sparse_readout(q, k, v, idx, 0.125, dropout_p=0.3, seed=5)
    b = sparse_readout(q, k, v, idx, 0.125, dropout_p=0.3, seed=5)
    c = sparse_readout(q, k, v, idx, 0.125, dropout_p=0.3, seed=6)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)
    z = sparse_readout(q, k, v, idx, 0.125, dropout_p=0.0, seed=5)
    assert torch.equal(z, sparse_readout(q, k, v, idx, 0.125))
    assert torch.count_nonzero(sparse_readout(q, k, v, idx, 0.125, dropout_p=1.0)) == 0


def test_module_training_forward_backward_with_dropout(device):
    """LearnedAddressSparseAttention (non-fused) in training mode: the HIP readout applies
    dropout; with torch.manual_seed the mask seed is known, and the output equals the
    oracle's dropout readout of the module's own q, k, v and retrieved indices."""
    from routing_attention.models import LearnedAddressSparseAttention

    _say("[dropout] module training forward + backward")
    torch.manual_seed(31)
    B, T, dm, H, K = 2, 256, 128, 4, 32
    m = LearnedAddressSparseAttention(dm, H, top_k=K, dropout=0.2).to(device).train()
    x = torch.randn(B, T, dm, device=device, requires_grad=True)
    torch.manual_seed(77)
    seed = draw_dropout_seed()
    torch.manual_seed(77)
    y = m(x)
    y.square().mean().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    # the indices as the forward retrieved them: with autograd on, the address projection is
    # torch's Linear (under no_grad it is the fused HIP projection, whose rounding differs)
    idx = m._retrieve_candidates(x).detach()
    with torch.no_grad():
        hd = dm // H
        q = m.q_proj(x).view(B, T, H, hd).transpose(1, 2)
        k = m.k_proj(x).view(B, T, H, hd).transpose(1, 2)
        v = m.v_proj(x).view(B, T, H, hd).transpose(1, 2)
    meat = native.sparse_readout_dropout(q.cpu(), k.cpu(), v.cpu(), idx.cpu(), hd ** -0.5, 0.2, seed)
    ref_y = m.out_proj.cpu().double()(meat.transpose(1, 2).reshape(B, T, dm))
    assert rel_err(y.detach(), ref_y) < 1e-4
