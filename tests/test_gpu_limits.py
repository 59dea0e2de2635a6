"""GPU parity at the edges of the drop-in interface: head dims that are not one of the lane
layouts' sizes (any D up to 256, multiples of 8 on the aligned kernels and any value on the
generic one), k_eff up to 512 and address dims up to 256 in the retrieval, and the readout
backward at D = 96 and 256 -- each against the oracle on the same seeded inputs.
The reference takes any D and K (fused_sparse.py:97-128, causal_topk.py:470-521); the
key-vector module searches with R = head_dim (attention.py:339-341)."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from oracle.readout_grad import grads_autograd
from routing_attention.kernels import fused_sparse_attention, sparse_meat_attention
from routing_attention.kernels.causal_topk import causal_topk_with_scores
from routing_attention.kernels.sparse_autograd import sparse_readout
from tests.helpers import addresses, qkv, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("D,dtype,layout", [
    (96, torch.bfloat16, "bthd"),     # aligned kernel, 12 of 16 lanes per neighbour
    (256, torch.bfloat16, "bthd"),    # aligned kernel, 32 lanes per neighbour
    (200, torch.float32, "bhtd"),     # aligned kernel, 25 of 32 lanes
    (8, torch.float16, "bhtd"),       # aligned kernel, 1 of 4 lanes
    (20, torch.bfloat16, "bhtd"),     # generic kernel: the head dim ends inside a slice
    (250, torch.float32, "bhtd"),     # generic kernel at the widest layout
])
def test_readout_any_head_dim(device, D, dtype, layout):
    _say(f"[limits] readout D={D} {dtype} {layout}")
    B, H, T, K = 2, 3, 300, 40
    g = torch.Generator().manual_seed(D)
    if layout == "bthd":
        q, k, v = (torch.randn(B, T, H, D, generator=g).to(dtype).transpose(1, 2) for _ in range(3))
    else:
        q, k, v = (torch.randn(B, H, T, D, generator=g).to(dtype) for _ in range(3))
    qa, ka = addresses(B, T, 32, seed=D + 1)
    idx = native.causal_topk(qa, ka, K)
    scale = D ** -0.5
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx.to(device), scale)
    ref = native.sparse_readout(q, k, v, idx, scale)
    assert got.shape == (B, H, T, D)
    assert rel_err(got.float(), ref) < TOL[dtype]


@pytest.mark.parametrize("D", [96, 256])
def test_readout_backward_wide_head_dims(device, D):
    _say(f"[limits] readout backward D={D}")
    B, H, T, K = 1, 2, 200, 24
    q, k, v = qkv(B, H, T, D, seed=D + 7, dtype=torch.float32)
    qa, ka = addresses(B, T, 32, seed=D + 8)
    idx = native.causal_topk(qa, ka, K)
    dout = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(D + 9))
    scale = D ** -0.5
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = sparse_readout(qd, kd, vd, idx.to(device), scale)
    out.backward(dout.to(device))
    ref_out = native.sparse_readout(q, k, v, idx, scale)
    assert rel_err(out.detach(), ref_out) < 1e-5
    _, rq, rk, rv = grads_autograd(q, k, v, idx, scale, dout)
    assert rel_err(qd.grad, rq) < 1e-5
    assert rel_err(kd.grad, rk) < 1e-5
    assert rel_err(vd.grad, rv) < 1e-5


@pytest.mark.parametrize("B,T,R,K,dtype", [
    (1, 1500, 32, 512, torch.bfloat16),     # k_eff 512
    (2, 900, 32, 300, torch.float32),       # 256 < k_eff < 512
    (1, 1200, 256, 128, torch.bfloat16),    # R = 256, aligned loads
    (1, 700, 200, 64, torch.float16),       # R = 200, element loads
    (1, 1000, 256, 400, torch.float32),     # both
])
def test_topk_wide_k_and_address_dim(device, B, T, R, K, dtype):
    _say(f"[limits] topk B={B} T={T} R={R} K={K} {dtype}")
    qa, ka = addresses(B, T, R, seed=T + R + K, dtype=dtype)
    idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
    torch.cuda.synchronize()
    ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
    bad = (idx.cpu() != ri).any(-1).nonzero()
    assert bad.numel() == 0, f"index mismatch at {bad[:6].tolist()}"
    assert torch.equal(sc.cpu(), rs)


def test_topk_k512_all_ties(device):
    _say("[limits] topk K=512 all ties")
    B, T, R, K = 1, 1300, 32, 512
    qa = torch.ones(B, T, R, dtype=torch.bfloat16)
    ka = torch.full((B, T, R), 0.25, dtype=torch.bfloat16)
    idx, _ = causal_topk_with_scores(qa.to(device), ka.to(device), K)
    assert torch.equal(idx.cpu(), native.causal_topk(qa, ka, K))
    assert idx[0, -1].tolist() == list(range(K))


def test_fused_head_dim_256_and_k512(device):
    _say("[limits] fused D=256 K=512")
    B, H, T, D, R, K = 1, 2, 1100, 256, 32, 512
    qa, ka = addresses(B, T, R, seed=91, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(92)
    q, k, v = (torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).transpose(1, 2) for _ in range(3))
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, D ** -0.5)
    ref_idx = native.causal_topk(qa, ka, K)
    assert torch.equal(idx.cpu(), ref_idx)
    assert rel_err(out.float(), native.sparse_readout(q, k, v, ref_idx, D ** -0.5)) < 2e-2


def test_key_vector_module_head_dim_256(device):
    """KeyVectorSparseAttention searches with R = head_dim: at head_dim 256 the retrieval runs
    with 256-dim search vectors (head means of q and k) on the HIP kernel."""
    from routing_attention.models import KeyVectorSparseAttention

    _say("[limits] key-vector module head_dim 256")
    torch.manual_seed(93)
    B, T, dm, H, K = 1, 400, 512, 2, 64
    m = KeyVectorSparseAttention(dm, H, top_k=K, dropout=0.0,
                                 retrieval_config={"use_fused_sparse": True}).to(device).eval()
    x = torch.randn(B, T, dm, device=device)
    with torch.no_grad():
        y = m(x)
        hd = dm // H
        q = m.q_proj(x).view(B, T, H, hd).transpose(1, 2)
        k = m.k_proj(x).view(B, T, H, hd).transpose(1, 2)
        v = m.v_proj(x).view(B, T, H, hd).transpose(1, 2)
        qs, ks = m._search_vectors(q, k)
    ref_idx = native.causal_topk(qs.cpu(), ks.cpu(), K)
    meat = native.sparse_readout(q.cpu(), k.cpu(), v.cpu(), ref_idx, hd ** -0.5)
    ref_y = m.out_proj.cpu().double()(meat.transpose(1, 2).reshape(B, T, dm))
    assert rel_err(y, ref_y) < 1e-4
