"""GPU parity of the retrieval on address patterns chosen to stress its speculative seed,
stretched pool checks and pruning, each bit-exact (indices and scores) against the oracle:

* rising  -- every key scores above all earlier ones for late queries: the K best are the
  most recent keys, so the last stretch of the prefix passes the seed at once (pools
  overflow and rows are screened again);
* falling -- the K best are the first keys: the seed, set from the whole prefix, is low
  for them and the first prune must do the work;
* clusters -- keys drawn around a few centres: large groups of near-equal scores;
* zero / constant keys -- every score equal (ties everywhere);
* huge and tiny magnitudes -- the error bound eps scales with max|k| (3e3 and 1e-15 times
  the normal addresses);
* planted -- sharp single winners;
* mixed shapes, batches, K and input types with the default seed settings.
* 128 < K <= 256 on random shapes, where the final selection runs inside the sort.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels.causal_topk import causal_topk_with_scores
from tests.helpers import addresses, plant

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _pattern(kind, B, T, R, seed):
    g = torch.Generator().manual_seed(seed)
    qa, ka = addresses(B, T, R, seed=seed)
    if kind == "rising":
        u = torch.ones(R) / R ** 0.5
        qa = qa * 0.1 + u
        ka = ka * 0.1 + u * torch.linspace(0, 4, T).view(1, T, 1)
    elif kind == "falling":
        u = torch.ones(R) / R ** 0.5
        qa = qa * 0.1 + u
        ka = ka * 0.1 + u * torch.linspace(4, 0, T).view(1, T, 1)
    elif kind == "clusters":
        centres = torch.randn(6, R, generator=g)
        pick = torch.randint(0, 6, (B, T), generator=g)
        ka = centres[pick] + 0.01 * torch.randn(B, T, R, generator=g)
    elif kind == "zero":
        ka = torch.zeros(B, T, R)
    elif kind == "huge":
        qa, ka = qa * 3.0e3, ka * 3.0e3
    elif kind == "tiny":
        qa, ka = qa * 1.0e-15, ka * 1.0e-15   # products stay normal floats
    elif kind == "planted":
        ka = plant(qa, ka, 0.02, seed=seed + 1)[0]
    return qa, ka


PATTERNS = [
    # kind, B, T, R, K, dtype
    ("rising", 1, 6000, 32, 128, torch.bfloat16),
    ("rising", 2, 3000, 32, 64, torch.float32),
    ("falling", 1, 6000, 32, 128, torch.bfloat16),
    ("falling", 1, 4000, 32, 256, torch.bfloat16),
    ("clusters", 1, 5000, 32, 128, torch.bfloat16),
    ("clusters", 2, 3000, 64, 100, torch.float16),
    ("zero", 1, 3000, 32, 128, torch.bfloat16),
    ("huge", 1, 5000, 32, 128, torch.bfloat16),
    ("tiny", 1, 3000, 32, 128, torch.float32),
    ("planted", 2, 4000, 32, 128, torch.bfloat16),
    ("planted", 1, 5000, 32, 512, torch.bfloat16),
]


@pytest.mark.parametrize("kind,B,T,R,K,dtype", PATTERNS)
def test_topk_patterns_match_oracle(device, kind, B, T, R, K, dtype):
    _say(f"[patterns] {kind} B{B} T{T} R{R} K{K} {dtype}")
    qa, ka = _pattern(kind, B, T, R, seed=T + K + R)
    qa, ka = qa.to(dtype), ka.to(dtype)
    idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
    torch.cuda.synchronize()
    ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
    bad = (idx.cpu() != ri).any(-1).nonzero()
    assert bad.numel() == 0, f"index mismatch at (b,t) {bad[:6].tolist()}"
    assert torch.equal(sc.cpu(), rs)


def test_topk_k256_select_in_sort(device):
    """Twelve shapes with 128 < K <= 256 and prefixes long enough that the final pools hold
    more than K entries, so the selection runs inside the sort (up to 64 entries past K in
    the last four lanes of a row) or, for fuller pools, through the radix select: B 1-2,
    T 600-9000, R in {32, 64}, every input type, normal or Student-t addresses."""
    g = torch.Generator().manual_seed(2027)
    dtypes = [torch.bfloat16, torch.float16, torch.float32]
    for i in range(12):
        B = int(torch.randint(1, 3, (1,), generator=g))
        T = int(torch.randint(600, 9001, (1,), generator=g))
        R = [32, 64][int(torch.randint(0, 2, (1,), generator=g))]
        K = int(torch.randint(129, 257, (1,), generator=g))
        dtype = dtypes[i % 3]
        dist = "student_t" if i % 2 else "normal"
        _say(f"[patterns] K256 {i}: B{B} T{T} R{R} K{K} {dtype} {dist}")
        qa, ka = addresses(B, T, R, seed=300 + i, dtype=dtype, dist=dist)
        idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
        torch.cuda.synchronize()
        ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
        bad = (idx.cpu() != ri).any(-1).nonzero()
        assert bad.numel() == 0, f"case {i}: index mismatch at (b,t) {bad[:6].tolist()}"
        assert torch.equal(sc.cpu(), rs), f"case {i}: scores differ"


def test_topk_random_shapes(device):
    """Twenty shapes drawn from a fixed generator: B 1-3, T 1-5000, R in {8, 24, 32, 64},
    K 1-300, every input type, normal or Student-t addresses."""
    g = torch.Generator().manual_seed(2026)
    dtypes = [torch.bfloat16, torch.float16, torch.float32]
    for i in range(20):
        B = int(torch.randint(1, 4, (1,), generator=g))
        T = int(torch.randint(1, 5001, (1,), generator=g))
        R = [8, 24, 32, 64][int(torch.randint(0, 4, (1,), generator=g))]
        K = int(torch.randint(1, 301, (1,), generator=g))
        dtype = dtypes[int(torch.randint(0, 3, (1,), generator=g))]
        dist = "student_t" if i % 3 == 2 else "normal"
        _say(f"[patterns] random {i}: B{B} T{T} R{R} K{K} {dtype} {dist}")
        qa, ka = addresses(B, T, R, seed=100 + i, dtype=dtype, dist=dist)
        idx, sc = causal_topk_with_scores(qa.to(device), ka.to(device), K)
        torch.cuda.synchronize()
        ri, rs = native.causal_topk(qa, ka, K, return_scores=True)
        bad = (idx.cpu() != ri).any(-1).nonzero()
        assert bad.numel() == 0, f"case {i}: index mismatch at (b,t) {bad[:6].tolist()}"
        assert torch.equal(sc.cpu(), rs), f"case {i}: scores differ"
