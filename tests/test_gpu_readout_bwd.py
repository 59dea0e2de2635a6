"""GPU parity of the readout backward (wf_sparse_readout_bwd through sparse_readout's
autograd) against the float64 gradient oracle (oracle/readout_grad.py).

Small shapes compare every gradient element with autograd of the reference's gather
formulation; the benchmark shape (config 4) checks two size-independent identities over
all elements plus sampled rows and keys against the closed-form oracle. Tolerance, norm-
wise ||a-b||_inf / ||b||_inf: 1e-5 fp32, 2e-3 fp16, 2e-2 bf16.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from oracle import readout_grad as rg
from routing_attention.kernels.sparse_autograd import sparse_readout
from tests.helpers import addresses, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(B, H, T, D, K, dtype, seed, idx_kind="topk", bthd=True):
    g = torch.Generator().manual_seed(seed)
    shape = (B, T, H, D) if bthd else (B, H, T, D)
    q, k, v, dout = (torch.randn(*shape, generator=g).to(dtype) for _ in range(4))
    if bthd:   # the module's (B, T, H, D) memory viewed as (B, H, T, D)
        q, k, v, dout = (t.transpose(1, 2) for t in (q, k, v, dout))
    if idx_kind == "topk":
        qa, ka = addresses(B, T, 32, seed=seed + 1)
        idx = native.causal_topk(qa, ka, K)
    elif idx_kind == "hub":   # skewed lists: 5/8 of every row's slots on six keys
        idx = torch.randint(0, T, (B, T, K), generator=g).to(torch.int32)
        nh = 5 * K // 8
        idx[:, :, :nh] = torch.randint(0, 6, (B, T, nh), generator=g).to(torch.int32) * 7
    else:      # arbitrary indices: duplicates, negative (wrap) and out-of-range (clamp)
        idx = torch.randint(-T, T + 3, (B, T, K), generator=g).to(torch.int32)
        idx[:, :, 1] = idx[:, :, 0]
    return q, k, v, dout, idx


def _hip_grads(q, k, v, dout, idx, scale, mask_pads, device):
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    out = sparse_readout(qd, kd, vd, idx.to(device), scale, mask_pads=mask_pads)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    return out.detach(), qd.grad, kd.grad, vd.grad


CASES = [
    # (B, H, T, D, K, dtype, idx_kind, mask_pads, bthd)
    (1, 4, 300, 64, 128, torch.float32, "topk", False, True),
    (2, 2, 513, 64, 37, torch.float32, "topk", True, True),
    (1, 2, 200, 32, 64, torch.float32, "random", False, False),
    (1, 2, 190, 128, 48, torch.float32, "topk", False, True),
    (2, 3, 257, 64, 128, torch.bfloat16, "topk", False, True),
    (1, 4, 400, 64, 16, torch.float16, "random", False, True),
    (1, 2, 150, 128, 100, torch.bfloat16, "random", True, False),
    # a few keys hold most entries: their lists are cut across the key pass's waves
    (1, 2, 600, 64, 64, torch.float32, "hub", False, True),
    (2, 2, 333, 128, 40, torch.float32, "hub", True, True),
    (1, 3, 700, 64, 96, torch.bfloat16, "hub", False, True),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[5]}-D{c[3]}-K{c[4]}-{c[6]}-mask{int(c[7])}" for c in CASES])
def test_readout_bwd_vs_autograd_oracle(device, case):
    B, H, T, D, K, dtype, kind, mask_pads, bthd = case
    _say(f"[bwd] B{B} H{H} T{T} D{D} K{K} {dtype} {kind} mask={mask_pads}")
    q, k, v, dout, idx = _inputs(B, H, T, D, K, dtype, seed=T + K, idx_kind=kind, bthd=bthd)
    scale = D ** -0.5
    out, dq, dk, dv = _hip_grads(q, k, v, dout, idx, scale, mask_pads, device)
    r_out, r_dq, r_dk, r_dv = rg.grads_autograd(q, k, v, idx, scale, dout, mask_pads)
    tol = TOL[dtype]
    assert rel_err(out.float(), r_out) < tol
    for name, a, b in (("dq", dq, r_dq), ("dk", dk, r_dk), ("dv", dv, r_dv)):
        assert a.dtype == dtype and a.shape == b.shape
        err = rel_err(a.float(), b)
        assert err < tol, f"{name} rel err {err:.3e}"


@pytest.mark.parametrize("kind", ["topk", "hub"])
def test_readout_bwd_deterministic(device, kind):
    _say(f"[bwd] determinism ({kind} indices)")
    q, k, v, dout, idx = _inputs(1, 4, 1024, 64, 128, torch.bfloat16, seed=11, idx_kind=kind)
    g1 = _hip_grads(q, k, v, dout, idx, 0.125, False, device)
    g2 = _hip_grads(q, k, v, dout, idx, 0.125, False, device)
    for a, b in zip(g1[1:], g2[1:]):
        assert torch.equal(a, b)


def test_readout_bwd_config4(device):
    """Config 4 shape (bf16, B1 H8 T16384 D64 K128), indices from the HIP retrieval."""
    _say("[bwd] config 4: bf16 B1 H8 T16384 D64 K128")
    from routing_attention.kernels import causal_topk

    B, H, T, D, K = 1, 8, 16384, 64, 128
    q, k, v, dout, _ = _inputs(B, H, T, D, 2, torch.bfloat16, seed=1004, idx_kind="random")
    qa, ka = addresses(B, T, 32, seed=2004, dtype=torch.bfloat16)
    idx = causal_topk(qa.to(device), ka.to(device), K)
    scale = D ** -0.5
    out, dq, dk, dv = _hip_grads(q, k, v, dout, idx, scale, False, device)
    f = lambda a, b: float((a.double() * b.double()).sum())  # noqa: E731
    qd, kd, vd, gd = (t.to(device) for t in (q, k, v, dout))
    # <dq,q> = <dk,k> and <dv,v> = <dout,out>, relative to the sum of |terms|
    lhs, rhs = f(dq, qd), f(dk, kd)
    mag = float((dq.double() * qd.double()).abs().sum())
    assert abs(lhs - rhs) <= 5e-3 * mag, (lhs, rhs, mag)
    lhs, rhs = f(dv, vd), f(gd, out)
    mag = float((dv.double() * vd.double()).abs().sum())
    assert abs(lhs - rhs) <= 5e-3 * mag, (lhs, rhs, mag)
    idx_c = idx.cpu()
    rows = [0, 1, 126, 127, 4097, 9999, 16383]
    ref = rg.dq_rows(q, k, v, idx_c, scale, dout, rows)
    assert rel_err(dq[:, :, rows].float(), ref) < 2e-2
    keys = [0, 5, 300, 8191, 16000, 16383]
    rk, rv = rg.dkdv_keys(q, k, v, idx_c, scale, dout, keys)
    assert rel_err(dk[:, :, keys].float(), rk) < 2e-2
    assert rel_err(dv[:, :, keys].float(), rv) < 2e-2


def test_module_training_step_grads(device):
    """LearnedAddressSparseAttention (non-fused, dropout 0) forward + backward on the HIP
    path: projection weight gradients against float64 autograd of the reference's layer
    (projections, gather readout, out_proj) on the same index sets."""
    from routing_attention.models import LearnedAddressSparseAttention

    _say("[bwd] module training step")
    torch.manual_seed(5)
    d_model, H, T, K = 128, 4, 256, 32
    m = LearnedAddressSparseAttention(d_model, H, top_k=K, dropout=0.0,
                                      retrieval_config={"dtype": "float32"}).to(device).train()
    x = torch.randn(2, T, d_model, generator=torch.Generator().manual_seed(6))
    y = m(x.to(device))
    (y.float() ** 2).sum().backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        qa, ka = m.address.forward_query_key(x.to(device))
        idx = native.causal_topk(qa.cpu(), ka.cpu(), K)
    # float64 reference of the same layer on the CPU
    sd = {n: p.detach().cpu().double().requires_grad_(True) for n, p in m.named_parameters()}
    xd = x.double()
    hd = d_model // H
    lin = lambda n, z: z @ sd[n + ".weight"].T + sd[n + ".bias"]  # noqa: E731
    q = lin("q_proj", xd).view(2, T, H, hd).transpose(1, 2)
    k = lin("k_proj", xd).view(2, T, H, hd).transpose(1, 2)
    v = lin("v_proj", xd).view(2, T, H, hd).transpose(1, 2)
    bi = torch.arange(2).view(2, 1, 1, 1)
    hi = torch.arange(H).view(1, H, 1, 1)
    ii = idx.long().unsqueeze(1)
    p = torch.softmax((q.unsqueeze(3) * k[bi, hi, ii]).sum(-1) * hd ** -0.5, dim=-1)
    meat = (p.unsqueeze(-1) * v[bi, hi, ii]).sum(3)
    ref = lin("out_proj", meat.transpose(1, 2).reshape(2, T, d_model))
    (ref ** 2).sum().backward()
    for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight", "out_proj.weight", "q_proj.bias"):
        got = dict(m.named_parameters())[n].grad
        err = rel_err(got, sd[n].grad)
        assert err < 1e-4, f"{n}: {err:.3e}"
