"""GPU parity of the sparse readout kernel (wf_sparse_readout_fwd) against the oracle's
double-precision readout on the same indices. Tolerances (norm-wise
||a-b||_inf / ||b||_inf): fp32 1e-5, bf16 2e-2, fp16 2e-3."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels import SparseMeatConfig, sparse_meat_attention
from tests.helpers import addresses, qkv, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [
    # B, H, T, D, K, dtype
    (1, 4, 2048, 64, 128, torch.float32),   # config 1 readout
    (1, 8, 1000, 64, 128, torch.bfloat16),
    (2, 3, 300, 32, 7, torch.float16),
    (1, 2, 500, 128, 256, torch.bfloat16),
    (3, 5, 64, 64, 1, torch.float32),
    (1, 4, 200, 128, 300, torch.float32),
    (2, 8, 129, 32, 128, torch.bfloat16),
]


@pytest.mark.parametrize("B,H,T,D,K,dtype", CASES)
def test_readout_matches_oracle(device, B, H, T, D, K, dtype):
    _say(f"[readout] B={B} H={H} T={T} D={D} K={K} {dtype}")
    q, k, v = qkv(B, H, T, D, seed=T + K + D, dtype=dtype)
    qa, ka = addresses(B, T, 32, seed=T * 3 + 1)
    if K <= T:
        idx = native.causal_topk(qa, ka, K)
    else:
        g = torch.Generator().manual_seed(K)
        idx = torch.randint(0, T, (B, T, K), generator=g, dtype=torch.int32)
    scale = D ** -0.5
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx.to(device), scale)
    torch.cuda.synchronize()
    ref = native.sparse_readout(q, k, v, idx, scale)
    assert got.dtype == dtype and got.shape == (B, H, T, D)
    err = rel_err(got.float(), ref)
    assert err < TOL[dtype], err


def test_readout_bthd_layout_and_strided_output(device):
    """q/k/v as .view(B,T,H,D).transpose(1,2) views (the module's layout), output into a
    (B,T,H,D)-memory view."""
    _say("[readout] (B,T,H,D) memory layout")
    B, H, T, D, K = 2, 8, 777, 64, 128
    g = torch.Generator().manual_seed(3)
    base = [torch.randn(B, T, H, D, generator=g).to(torch.bfloat16) for _ in range(3)]
    q, k, v = (x.to(device).transpose(1, 2) for x in base)
    qa, ka = addresses(B, T, 32, seed=4)
    idx = native.causal_topk(qa, ka, K)
    got = sparse_meat_attention(q, k, v, idx.to(device), 0.125)
    ref = native.sparse_readout(*(x.transpose(1, 2) for x in base), idx, 0.125)
    assert rel_err(got.float(), ref) < 2e-2


def test_readout_duplicates_negative_and_out_of_range(device):
    _say("[readout] duplicates / negative / clamped indices")
    B, H, T, D, K = 1, 2, 300, 64, 40
    q, k, v = qkv(B, H, T, D, seed=5)
    g = torch.Generator().manual_seed(6)
    idx = torch.randint(-T, 2 * T, (B, T, K), generator=g, dtype=torch.int32)
    idx[..., :5] = 17                                        # duplicates
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx.to(device), 0.2)
    ref = native.sparse_readout(q, k, v, idx, 0.2)
    assert rel_err(got, ref) < 1e-5


def test_readout_mask_pads(device):
    _say("[readout] mask_pads")
    B, H, T, D, K = 1, 4, 400, 64, 128
    q, k, v = qkv(B, H, T, D, seed=7)
    qa, ka = addresses(B, T, 32, seed=8)
    idx = native.causal_topk(qa, ka, K)
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx.to(device), 0.125,
                                config=SparseMeatConfig(mask_pads=True))
    ref = native.sparse_readout(q, k, v, idx, 0.125, flags=1)
    assert rel_err(got, ref) < 1e-5
    # masked row t reads only keys <= t: row 0 is v[.., 0]
    assert torch.allclose(got[:, :, 0].cpu(), v[:, :, 0], atol=1e-6)


def test_readout_int64_indices_and_empty(device):
    _say("[readout] int64 indices, K=0")
    B, H, T, D = 1, 2, 50, 32
    q, k, v = qkv(B, H, T, D, seed=9)
    idx = torch.randint(0, T, (B, T, 6), dtype=torch.int64)
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx.to(device), 0.3)
    assert rel_err(got, native.sparse_readout(q, k, v, idx, 0.3)) < 1e-5
    z = sparse_meat_attention(q.to(device), k.to(device), v.to(device),
                              torch.zeros(B, T, 0, dtype=torch.int32, device=device), 0.3)
    assert torch.count_nonzero(z) == 0
