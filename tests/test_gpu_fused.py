"""GPU parity of the fused entry point (wf_fused_topk_sparse_fwd) and of the drop-in
LearnedAddressSparseAttention module against the oracle, at the benchmark configs."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels import fused_sparse_attention
from routing_attention.models import LearnedAddressSparseAttention
from tests.helpers import addresses, plant, qkv, rel_err

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fused_vs_oracle(device, B, H, T, D, R, K, dtype, seed, tol, ka_fn=None):
    qa, ka = addresses(B, T, R, seed=seed, dtype=torch.float32)
    if ka_fn is not None:
        ka = ka_fn(qa, ka)
    qa, ka = qa.to(dtype), ka.to(dtype)
    q, k, v = qkv(B, H, T, D, seed=seed + 1, dtype=dtype)
    scale = D ** -0.5
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, scale)
    torch.cuda.synchronize()
    ref_idx = native.causal_topk(qa, ka, K)
    bad = (idx.cpu() != ref_idx).any(-1).nonzero()
    assert bad.numel() == 0, f"index mismatch at {bad[:6].tolist()}"
    ref_out = native.sparse_readout(q, k, v, ref_idx, scale)
    err = rel_err(out.float(), ref_out)
    assert out.dtype == dtype and err < tol, err
    return err


def test_fused_config1_fp32(device):
    _say("[fused] config 1: fp32 B1 H4 T2048 D64 K128")
    _fused_vs_oracle(device, 1, 4, 2048, 64, 32, 128, torch.float32, 1001, 1e-5)


def test_fused_config3_planted_bf16(device):
    _say("[fused] config 3: bf16 B4 H8 T4096 planted")
    _fused_vs_oracle(device, 4, 8, 4096, 64, 32, 128, torch.bfloat16, 1003, 2e-2,
                     ka_fn=lambda qa, ka: plant(qa, ka, 0.01, seed=2003)[0])


def test_fused_config4_bf16(device):
    _say("[fused] config 4: bf16 B1 H8 T16384 D64 K128")
    _fused_vs_oracle(device, 1, 8, 16384, 64, 32, 128, torch.bfloat16, 1004, 2e-2)


def test_fused_fp16_long_rows(device):
    """fp16 addresses and q/k/v, K not a power of two, prefixes long enough for the seeded
    screen (T = 6000)."""
    _say("[fused] fp16 B2 H4 T6000 D64 K100")
    _fused_vs_oracle(device, 2, 4, 6000, 64, 32, 100, torch.float16, 1006, 2e-3)


def test_fused_short_and_odd_shapes(device):
    _say("[fused] odd shapes")
    _fused_vs_oracle(device, 2, 3, 77, 32, 16, 128, torch.float16, 11, 2e-3)
    _fused_vs_oracle(device, 1, 2, 1, 128, 32, 4, torch.float32, 12, 1e-5)


def test_module_fused_path_matches_oracle(device):
    """Drop-in module: projections on the GPU, then the fused HIP path; the oracle sees the
    same projected tensors."""
    _say("[module] LearnedAddressSparseAttention fused path")
    torch.manual_seed(0)
    B, T, dm, H, K = 2, 700, 256, 4, 128
    m = LearnedAddressSparseAttention(dm, H, top_k=K, address_dim=32, dropout=0.0,
                                      retrieval_config={"use_fused_sparse": True}).to(device).eval()
    x = torch.randn(B, T, dm, device=device)
    with torch.no_grad():
        y, attn = m(x, return_attention=True)
        hd = dm // H
        q = m.q_proj(x).view(B, T, H, hd).transpose(1, 2)
        k = m.k_proj(x).view(B, T, H, hd).transpose(1, 2)
        v = m.v_proj(x).view(B, T, H, hd).transpose(1, 2)
        qa, ka = m.address.forward_query_key(x)
    ref_idx = native.causal_topk(qa.cpu(), ka.cpu(), K)
    meat = native.sparse_readout(q.cpu(), k.cpu(), v.cpu(), ref_idx, hd ** -0.5)
    ref_y = m.out_proj.cpu().double()(meat.transpose(1, 2).reshape(B, T, dm))
    assert rel_err(y, ref_y) < 1e-4
    assert torch.allclose(attn.sum(-1).cpu()[:, K:], torch.ones(B, T - K))


def test_module_unfused_eval_path(device):
    _say("[module] unfused eval path (float16 retrieval + HIP readout)")
    torch.manual_seed(1)
    B, T, dm, H, K = 1, 300, 128, 2, 32
    m = LearnedAddressSparseAttention(dm, H, top_k=K, dropout=0.0).to(device).eval()
    x = torch.randn(B, T, dm, device=device)
    with torch.no_grad():
        y = m(x)
        hd = dm // H
        qa, ka = m.address.forward_query_key(x)
        q = m.q_proj(x).view(B, T, H, hd).transpose(1, 2)
        k = m.k_proj(x).view(B, T, H, hd).transpose(1, 2)
        v = m.v_proj(x).view(B, T, H, hd).transpose(1, 2)
    idx = native.causal_topk(qa.cpu().half(), ka.cpu().half(), K)
    meat = native.sparse_readout(q.cpu(), k.cpu(), v.cpu(), idx, hd ** -0.5)
    ref_y = m.out_proj.cpu().double()(meat.transpose(1, 2).reshape(B, T, dm))
    assert rel_err(y, ref_y) < 1e-4
