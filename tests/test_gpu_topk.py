"""GPU parity of the causal top-K kernel (wf_causal_topk_fwd via the Python drop-in) against
the CPU oracle on identical seeded inputs: indices and fp32 scores must match bit-exactly
(canonical order: score descending, ties to the lower index, pads last)."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels import causal_topk, causal_topk_reference
from routing_attention.kernels.causal_topk import causal_topk_with_scores
from tests.helpers import addresses, plant

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check_exact(qa, ka, K, device, rows=None):
    idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
    torch.cuda.synchronize()
    idx, sc = idx.cpu(), sc.cpu()
    if rows is None:
        ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
        bad = (idx != ri).any(-1).nonzero()
        assert bad.numel() == 0, f"index mismatch at (b,t) {bad[:6].tolist()}"
        assert torch.equal(sc, rs)
    else:
        for b, r0, r1 in rows:
            ri, rs = native.causal_topk_rows(qa, ka, K, b, r0, r1, return_scores=True)
            bad = (idx[b, r0:r1] != ri).any(-1).nonzero()
            assert bad.numel() == 0, f"index mismatch at b={b} rows {(bad[:6] + r0).tolist()}"
            assert torch.equal(sc[b, r0:r1], rs)
    return idx, sc


CASES = [
    # B, T, R, K, dtype
    (1, 1, 32, 128, torch.bfloat16),
    (1, 2, 32, 128, torch.bfloat16),
    (2, 15, 32, 8, torch.float32),
    (1, 16, 32, 16, torch.bfloat16),
    (1, 17, 32, 16, torch.float16),
    (3, 100, 32, 64, torch.bfloat16),
    (1, 130, 32, 128, torch.bfloat16),
    (2, 300, 32, 128, torch.float32),
    (1, 1000, 64, 128, torch.bfloat16),
    (1, 777, 24, 50, torch.bfloat16),      # R not a multiple of 8: element loads
    (1, 500, 128, 256, torch.float32),
    (1, 600, 16, 1, torch.bfloat16),
    (2, 1500, 32, 200, torch.float16),
    (1, 2048, 32, 128, torch.float32),      # config 1 retrieval
]


@pytest.mark.parametrize("B,T,R,K,dtype", CASES)
def test_topk_matches_oracle(device, B, T, R, K, dtype):
    _say(f"[topk] B={B} T={T} R={R} K={K} {dtype}")
    qa, ka = addresses(B, T, R, seed=B * 100003 + T * 31 + K, dtype=dtype)
    _check_exact(qa, ka, K, device)


def test_topk_strided_inputs(device):
    _say("[topk] strided inputs")
    B, T, R, K = 2, 400, 32, 64
    qa, ka = addresses(B, T, 2 * R, seed=5, dtype=torch.bfloat16)
    qs, ks = qa[..., ::2], ka[..., 1::2]                       # element stride 2
    idx_g, _ = causal_topk_with_scores(qs.to(device), ks.to(device), K)
    ref = native.causal_topk(qs.contiguous(), ks.contiguous(), K)
    assert torch.equal(idx_g.cpu(), ref)
    qt = qa[..., :R].contiguous().transpose(1, 2).contiguous().transpose(1, 2)  # (B,T,R) view of (B,R,T)
    idx_t = causal_topk(qt.to(device), ka[..., :R].to(device), K)
    assert torch.equal(idx_t.cpu(), native.causal_topk(qa[..., :R], ka[..., :R], K))


def test_topk_sliding_window(device):
    _say("[topk] sliding window")
    B, T, R, K = 1, 700, 32, 128
    qa = torch.zeros(B, T, R)
    qa[..., 0] = 1.0
    ka = torch.zeros(B, T, R)
    ka[0, :, 0] = torch.arange(T, dtype=torch.float32) / T
    idx, _ = _check_exact(qa, ka, K, device)
    for t in (0, 5, 127, 128, 699):
        n = min(K, t + 1)
        assert idx[0, t, :n].tolist() == list(range(t, t - n, -1))


@pytest.mark.parametrize("K,T", [(128, 900), (256, 1500), (200, 1200)])
def test_topk_all_ties(device, K, T):
    """Every score equal: the lower-index rule selects keys 0..K-1 in every full row (the
    pools never shrink, so the exact path runs in the loop)."""
    _say(f"[topk] all ties K={K} T={T}")
    B, R = 1, 32
    qa = torch.ones(B, T, R, dtype=torch.bfloat16)
    ka = torch.full((B, T, R), 0.25, dtype=torch.bfloat16)
    idx, _ = _check_exact(qa, ka, K, device)
    assert idx[0, -1].tolist() == list(range(K))


@pytest.mark.parametrize("K,T", [(128, 3000), (100, 2500), (256, 3000), (200, 2600)])
def test_topk_quantized_score_ties(device, K, T):
    """Addresses in {-1, 0, 1}: every score is a small integer, so each row's K-th place
    falls inside a large group of equal scores and the lower-index rule decides the set.
    Covers the final selection fused into the sort (64 < K <= 128, pools of K..K+16
    entries), the radix select with 20 and 32 entries per lane (K in (128, 256]) and the
    in-loop exact path that runs when ties keep a pool from shrinking."""
    _say(f"[topk] quantized ties K={K} T={T}")
    g = torch.Generator().manual_seed(4242 + K)
    B, R = 2, 32
    qa = torch.randint(-1, 2, (B, T, R), generator=g).to(torch.bfloat16)
    ka = torch.randint(-1, 2, (B, T, R), generator=g).to(torch.bfloat16)
    _check_exact(qa, ka, K, device)


def test_topk_short_sequence_wraps_pads(device):
    _say("[topk] T < K")
    qa, ka = addresses(2, 50, 32, seed=8, dtype=torch.bfloat16)
    idx, _ = _check_exact(qa, ka, 128, device)
    assert idx.shape == (2, 50, 50)


def test_topk_planted_config3(device):
    """Config 3 retrieval: B=4, T=4096, bf16, 1% of keys planted as 4x copies of a later
    query address; every planted key is retrieved by its query."""
    _say("[topk] config 3 planted")
    qa, ka = addresses(4, 4096, 32, seed=1003, dtype=torch.float32)
    ka, plants = plant(qa, ka, 0.01, seed=2003)
    qa, ka = qa.to(torch.bfloat16), ka.to(torch.bfloat16)
    idx, _ = _check_exact(qa, ka, 128, device)
    for b, i, j in plants:
        assert j in idx[b, i].tolist()


def test_topk_config4_full(device):
    """Headline shape, every row against the oracle."""
    _say("[topk] config 4 full T=16384")
    qa, ka = addresses(1, 16384, 32, seed=1004, dtype=torch.bfloat16)
    _check_exact(qa, ka, 128, device)


def test_topk_config5_heavy_tail_sampled(device):
    """Long-context stretch: T=65536, K=256, Student-t(3) addresses; sampled row ranges."""
    _say("[topk] config 5 T=65536 K=256 student-t")
    qa, ka = addresses(1, 65536, 32, seed=1005, dtype=torch.bfloat16, dist="student_t")
    rows = [(0, 0, 300), (0, 30000, 30032), (0, 65536 - 48, 65536)]
    _check_exact(qa, ka, 256, device, rows=rows)


@pytest.mark.parametrize("K,dtype", [(256, torch.bfloat16), (100, torch.float32), (64, torch.float16)])
def test_topk_heavy_tail_full(device, K, dtype):
    """Student-t(3) addresses on every row: a few large keys stretch each pool's score range,
    which sends the pruning to its second, order-preserving histogram (and the exact fallback
    when scores crowd); indices and scores must still equal the oracle's."""
    _say(f"[topk] heavy tail full T=6000 K={K} {dtype}")
    qa, ka = addresses(2, 6000, 32, seed=4000 + K, dtype=torch.float32, dist="student_t")
    _check_exact(qa.to(dtype), ka.to(dtype), K, device)


def test_topk_deterministic(device):
    _say("[topk] determinism")
    qa, ka = addresses(2, 3000, 32, seed=77, dtype=torch.bfloat16)
    a = causal_topk(qa.to(device), ka.to(device), 128)
    b = causal_topk(qa.to(device), ka.to(device), 128)
    assert torch.equal(a, b)


def test_topk_dtype_argument_and_reference_api(device):
    _say("[topk] dtype= and causal_topk_reference")
    qa, ka = addresses(1, 300, 32, seed=9)
    got = causal_topk(qa.to(device), ka.to(device), 64, dtype="float16")
    assert torch.equal(got.cpu(), native.causal_topk(qa.half(), ka.half(), 64))
    ref = causal_topk_reference(qa.to(device), ka.to(device), 64)
    assert torch.equal(ref.cpu(), native.causal_topk(qa, ka, 64))
