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


def _lse2_reference(q, k, idx, scale):
    """Base-2 log-sum-exp of every (b, h, t) row in float64: log2(sum_s exp(scale q.k_s))."""
    B, H, T, D = q.shape
    j = idx.long()
    j = torch.where(j < 0, j + T, j).clamp(0, T - 1)
    ks = k.double()[torch.arange(B).view(B, 1, 1, 1), torch.arange(H).view(1, H, 1, 1), j.unsqueeze(1)]
    sc = (q.double().unsqueeze(-2) * ks).sum(-1) * scale
    return torch.logsumexp(sc, dim=-1) / torch.log(torch.tensor(2.0, dtype=torch.float64))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_readout_generic_kernel_strided_indices(device, dtype):
    """Index rows with element stride 2 leave the aligned fast kernel: the generic kernel
    reads every index through its strides. Output and the training forward's lse2."""
    from routing_attention.kernels.sparse_autograd import readout_fwd_lse

    _say(f"[readout] generic kernel, index stride 2, {dtype}")
    B, H, T, D, K = 2, 3, 333, 64, 48
    q, k, v = qkv(B, H, T, D, seed=21, dtype=dtype)
    g = torch.Generator().manual_seed(22)
    wide = torch.randint(-T, T, (B, T, 2 * K), generator=g, dtype=torch.int32)
    idx_dev = wide.to(device)[..., ::2]
    assert idx_dev.stride(-1) == 2
    idx = wide[..., ::2].contiguous()
    scale = D ** -0.5
    got = sparse_meat_attention(q.to(device), k.to(device), v.to(device), idx_dev, scale)
    ref = native.sparse_readout(q, k, v, idx, scale)
    assert rel_err(got.float(), ref) < TOL[dtype]
    out, lse2 = readout_fwd_lse(q.to(device), k.to(device), v.to(device), idx_dev, scale)
    assert rel_err(out.float(), ref) < TOL[dtype]
    lref = _lse2_reference(q, k, idx, scale)
    assert (lse2.cpu().double() - lref).abs().max().item() < (1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 32), (torch.float32, 128)])
def test_readout_generic_kernel_unaligned_qkv(device, dtype, D):
    """q/k/v views starting one element into their storage: rows are not 16-byte aligned, so
    the generic kernel's element loads run (VEC off), output into an unaligned view too."""
    from routing_attention.kernels.sparse_autograd import readout_fwd_lse

    _say(f"[readout] generic kernel, odd element offset, {dtype} D={D}")
    B, H, T, K = 1, 2, 257, 33
    n = B * H * T * D
    g = torch.Generator().manual_seed(23)
    stores = [torch.randn(n + 1, generator=g).to(dtype) for _ in range(3)]
    q, k, v = (s[1:].view(B, H, T, D) for s in stores)
    qa, ka = addresses(B, T, 32, seed=24)
    idx = native.causal_topk(qa, ka, K)
    dq, dk, dv = (s.to(device)[1:].view(B, H, T, D) for s in stores)
    assert dq.data_ptr() % 16 != 0
    out_store = torch.empty(n + 1, dtype=dtype, device=device)
    out = out_store[1:].view(B, H, T, D)
    idx_dev = idx.to(device)
    scale = 0.17
    from routing_attention.kernels import _lib
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.wf_sparse_readout_fwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), _lib.dtype_code(dq),
                                       B, H, T, D, _lib.strides(dq), _lib.strides(dk), _lib.strides(dv),
                                       idx_dev.data_ptr(), _lib.strides(idx_dev), K, scale, 0,
                                       out.data_ptr(), _lib.strides(out), _lib.stream_ptr(device))
    _lib.check(rc)
    torch.cuda.synchronize()
    ref = native.sparse_readout(q, k, v, idx, scale)
    assert rel_err(out.float(), ref) < TOL[dtype]
    out2, lse2 = readout_fwd_lse(dq, dk, dv, idx_dev, scale)
    assert rel_err(out2.float(), ref) < TOL[dtype]
    lref = _lse2_reference(q, k, idx, scale)
    assert (lse2.cpu().double() - lref).abs().max().item() < (1e-4 if dtype == torch.float32 else 1e-2)
