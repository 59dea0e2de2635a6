"""GPU parity of the retrieval's speculative seed. Each row block screens with a threshold
estimated from a sample of its key prefix, checks every row exactly afterwards, and screens a
row's prefix again (keeping its pool) when the check fails: for the band of MFMA scores just
below the seed when the row kept K keys, for every key below the seed when it kept fewer.

WAYFINDER_TOPK_SEED_ALPHA sets how many keys (alpha * K) the seed aims to let through; the
library reads it at every launch. alpha = 1.01 sets the seed near each row's K-th score, so
about half of the seeded rows fail the check and take one of the two fallback branches; the
results must still equal the oracle's bit for bit, as they must with the seed off (alpha 0)
and at the default. Covered: both fallback branches, ties (every seeded row fails with K
kept), heavy tails, every retrieval kernel shape (K <= 128 fused sort-merge, K = 256 radix
select, K = 512 wide kernel, R = 64, element loads) and the single-pass fused kernel, whose
LDS index rows must not overwrite the pool of a row that fails."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels import SparseMeatConfig, fused_sparse_attention
from routing_attention.kernels.causal_topk import causal_topk_with_scores
from tests.helpers import addresses, rel_err

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture
def alpha(monkeypatch):
    def set_alpha(a):
        if a is None:
            monkeypatch.delenv("WAYFINDER_TOPK_SEED_ALPHA", raising=False)
        else:
            monkeypatch.setenv("WAYFINDER_TOPK_SEED_ALPHA", str(a))
    return set_alpha


def _inputs(kind, B, T, R, dtype, seed):
    if kind == "normal":
        return addresses(B, T, R, seed=seed, dtype=dtype)
    if kind == "student_t":
        return addresses(B, T, R, seed=seed, dtype=dtype, dist="student_t")
    g = torch.Generator().manual_seed(seed)
    if kind == "quantized":      # scores are small integers: large groups of equal scores
        qa = torch.randint(-1, 2, (B, T, R), generator=g)
        ka = torch.randint(-1, 2, (B, T, R), generator=g)
        return qa.to(dtype), ka.to(dtype)
    if kind == "ties":           # every score equal
        return torch.ones(B, T, R, dtype=dtype), torch.full((B, T, R), 0.25, dtype=dtype)
    raise ValueError(kind)


def _check(qa, ka, K, device):
    idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
    torch.cuda.synchronize()
    ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
    bad = (idx.cpu() != ri).any(-1).nonzero()
    assert bad.numel() == 0, f"index mismatch at (b,t) {bad[:6].tolist()}"
    assert torch.equal(sc.cpu(), rs)
    return idx


CASES = [
    # kind, alpha, B, T, R, K, dtype, note
    ("normal", 1.01, 1, 4096, 32, 128, torch.bfloat16, "both branches, fused sort-merge select"),
    ("normal", 1.3, 2, 3000, 32, 64, torch.float32, "fp32 operands"),
    ("normal", 0, 1, 4096, 32, 128, torch.bfloat16, "seed off"),
    ("normal", None, 1, 5000, 32, 100, torch.float16, "default alpha"),
    ("student_t", 1.05, 1, 6000, 32, 256, torch.bfloat16, "heavy tail, K = 256 radix select"),
    ("student_t", None, 1, 6000, 32, 256, torch.bfloat16, "heavy tail, default alpha"),
    ("quantized", 1.01, 1, 4000, 32, 100, torch.bfloat16, "ties at the seed"),
    ("ties", None, 1, 4096, 32, 32, torch.bfloat16, "all equal: every seeded row fails with K kept"),
    ("normal", 1.01, 1, 6000, 32, 512, torch.bfloat16, "wide kernel, K = 512"),
    ("normal", 1.01, 1, 3000, 64, 128, torch.bfloat16, "R = 64"),
    ("normal", 1.01, 1, 3000, 24, 128, torch.bfloat16, "R = 24, element loads"),
]


@pytest.mark.parametrize("kind,a,B,T,R,K,dtype,note", CASES)
def test_seeded_topk_matches_oracle(device, alpha, kind, a, B, T, R, K, dtype, note):
    _say(f"[seed] {kind} alpha={a} B{B} T{T} R{R} K{K} {dtype} ({note})")
    alpha(a)
    qa, ka = _inputs(kind, B, T, R, dtype, seed=T + K + R)
    idx = _check(qa, ka, K, device)
    if kind == "ties":
        assert idx[0, -1].tolist() == list(range(K))


@pytest.mark.parametrize("T,lo,hi,K", [(8192, 5000, 5600, 128), (16384, 9000, 10200, 64), (12000, 2000, 2600, 100)])
def test_burst_overflows_stretched_checks(device, alpha, T, lo, hi, K):
    """A run of keys aligned with every query: nearly all of them pass the seed within one
    stretched check interval, so pools overflow (appends stay inside the pool, the count
    shows it) and those rows are screened again from -inf with worst-case checks."""
    _say(f"[seed] burst keys {lo}..{hi} of T={T}, K={K}")
    alpha(None)
    B, R = 1, 32
    qa, ka = addresses(B, T, R, seed=T + lo, dtype=torch.float32)
    mu = torch.ones(R) / R ** 0.5
    qa = qa + 0.5 * mu
    ka[:, lo:hi] = ka[:, lo:hi] + 1.5 * mu
    _check(qa.to(torch.bfloat16), ka.to(torch.bfloat16), K, device)


def test_seeded_topk_repeatable_across_alphas(device, alpha):
    """The seed changes the work, never the result: the same indices at every alpha."""
    _say("[seed] identical indices at alpha 0, 1.01, 2, default")
    qa, ka = _inputs("normal", 2, 3500, 32, torch.bfloat16, seed=77)
    outs = []
    for a in (0, 1.01, 2, None):
        alpha(a)
        idx, _ = causal_topk_with_scores(qa.to(device), ka.to(device), 128)
        outs.append(idx.cpu())
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("mode", ["single", "split"])
def test_burst_overflow_fused_paths(device, alpha, mode):
    """Rows whose pools overflow in pass 0 through the fused forward: the single-pass kernel
    must not read out a row before pass 1 has retrieved it again."""
    _say(f"[seed] fused {mode}, burst keys")
    alpha(None)
    B, H, T, D, K, R = 1, 8, 8192, 64, 128, 32
    qa, ka = addresses(B, T, R, seed=8192 + 5000, dtype=torch.float32)
    mu = torch.ones(R) / R ** 0.5
    qa = (qa + 0.5 * mu).to(torch.bfloat16)
    ka[:, 5000:5600] = ka[:, 5000:5600] + 1.5 * mu
    ka = ka.to(torch.bfloat16)
    g = torch.Generator().manual_seed(503)
    q, k, v = (torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).transpose(1, 2) for _ in range(3))
    cfg = SparseMeatConfig(fused_pass=mode)
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, D ** -0.5, meat_config=cfg)
    torch.cuda.synchronize()
    ref_idx = native.causal_topk(qa, ka, K)
    assert torch.equal(idx.cpu(), ref_idx)
    assert rel_err(out.float(), native.sparse_readout(q, k, v, ref_idx, D ** -0.5)) < 2e-2


@pytest.mark.parametrize("mode", ["single", "split"])
def test_seeded_fused_paths(device, alpha, mode):
    """Fused forward with seeds that fail often: the single-pass kernel reads each row's
    indices from LDS after the retrieval, so a failed row's pool must survive pass 0."""
    _say(f"[seed] fused {mode} alpha=1.01")
    alpha(1.01)
    B, H, T, D, K = 1, 8, 4096, 64, 128
    qa, ka = _inputs("normal", B, T, 32, torch.bfloat16, seed=501)
    g = torch.Generator().manual_seed(502)
    q, k, v = (torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).transpose(1, 2) for _ in range(3))
    cfg = SparseMeatConfig(fused_pass=mode)
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, D ** -0.5, meat_config=cfg)
    torch.cuda.synchronize()
    ref_idx = native.causal_topk(qa, ka, K)
    assert torch.equal(idx.cpu(), ref_idx)
    assert rel_err(out.float(), native.sparse_readout(q, k, v, ref_idx, D ** -0.5)) < 2e-2
