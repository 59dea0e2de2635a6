"""Full-size parity of the fused path and a cross-check against torch's own arithmetic.

* Config 5 (B1 H8 T65536 D128 K256, bf16, Student-t(3) addresses): the fused entry point
  at full size, indices and outputs compared with the C oracle on 2,048+ rows (rows
  0..299, the last 64, and a seeded random set in between).
* Configs 3/4/5 against the reference's GPU arithmetic: oracle/torch_reference
  .row_blocked_topk run on the device tensors -- torch's own fp32 bmm and
  topk(sorted=False) in row blocks, then the reference's pad finalisation. On rows
  t >= K-1 every index difference must be a near-tie of the K-th score (within the
  rounding bound of two fp32 dot products of length R); the number of differing rows is
  printed. On rows t < K-1 the whole slot set, pads included, must equal torch's: the pad
  indices depend on where topk(sorted=False) leaves the valid entries.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from oracle import torch_reference as tr
from routing_attention.kernels import (
    causal_topk_available,
    fused_sparse_attention,
    fused_sparse_attention_available,
)
from routing_attention.kernels.causal_topk import causal_topk, causal_topk_with_scores
from tests.helpers import addresses, plant, rel_err

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _bthd(B, T, H, D, seed, dtype):
    """q, k, v as (B, H, T, D) views of (B, T, H, D) memory (the module's layout)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, T, H, D, generator=g).to(dtype).transpose(1, 2) for _ in range(3)]


def test_availability_probes_on_gpu(device):
    assert causal_topk_available() and fused_sparse_attention_available()


def test_fused_zero_heads_still_retrieves(device):
    """H == 0: no readout, but the indices are still the causal top-K (the reference
    computes them before the readout)."""
    _say("[fused] H=0")
    B, T, R, K = 2, 300, 32, 64
    qa, ka = addresses(B, T, R, seed=31, dtype=torch.bfloat16)
    z = torch.empty(B, 0, T, 64, dtype=torch.bfloat16, device=device)
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), z, z, z, K, 0.125)
    assert out.shape == (B, 0, T, 64)
    assert torch.equal(idx.cpu(), native.causal_topk(qa, ka, K))


def test_fused_config5_full_size(device):
    """Config 5 at full size: B1 H8 T65536 D128 K256, bf16, Student-t(3) addresses."""
    B, H, T, D, R, K = 1, 8, 65536, 128, 32, 256
    _say(f"[fused] config 5 full: B{B} H{H} T{T} D{D} K{K} bf16 student-t")
    qa, ka = addresses(B, T, R, seed=1005, dtype=torch.bfloat16, dist="student_t")
    q, k, v = _bthd(B, T, H, D, 2005, torch.bfloat16)
    scale = D ** -0.5
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, scale)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(3005)
    middle = torch.randperm(T - 364, generator=g)[:1700] + 300
    ts = torch.cat([torch.arange(300), middle.sort().values, torch.arange(T - 64, T)])
    rows = torch.stack([torch.zeros_like(ts), ts], dim=1)
    _say(f"[fused] config 5: checking {rows.shape[0]} rows against the oracle")
    ref_idx = native.causal_topk_rowlist(qa, ka, K, rows)
    got_idx = idx.cpu()[0, ts]
    bad = (got_idx != ref_idx).any(-1).nonzero()
    assert bad.numel() == 0, f"index mismatch at rows {ts[bad[:6, 0]].tolist()}"
    ref_out = native.sparse_readout_rows(q, k, v, rows, ref_idx, scale)    # (n, H, D)
    got_out = out.cpu()[0, :, ts].transpose(0, 1).float()                # (n, H, D)
    err = rel_err(got_out, ref_out)
    _say(f"[fused] config 5 output rel err {err:.3e} on {rows.shape[0]} rows")
    assert err < 2e-2


def _near_tie_bound(q: torch.Tensor, kmax: float) -> torch.Tensor:
    """Per row: 4 x the bound R 2^-23 ||q||_1 max|k| on the error of an fp32 dot product of
    length R in any summation order (torch's bmm and the kernel's FMA chain each carry
    one; the comparison sees both twice over)."""
    R = q.shape[-1]
    return 4.0 * R * 2.0 ** -23 * q.double().abs().sum(-1) * kmax


@pytest.mark.parametrize("cfg", ["c3", "c4", "c5"])
def test_index_sets_vs_torch_gpu_topk(device, cfg):
    B, T, R, K, dist, seed = {"c3": (4, 4096, 32, 128, "normal", 1003),
                              "c4": (1, 16384, 32, 128, "normal", 1004),
                              "c5": (1, 65536, 32, 256, "student_t", 1005)}[cfg]
    _say(f"[crosscheck] {cfg}: B{B} T{T} K{K} {dist} vs torch bmm + topk(sorted=False) on the GPU")
    qa, ka = addresses(B, T, R, seed=seed, dtype=torch.float32, dist=dist)
    if cfg == "c3":
        ka = plant(qa, ka, 0.01, seed=2003)[0]
    qa, ka = qa.to(torch.bfloat16), ka.to(torch.bfloat16)
    qd, kd = qa.to(device), ka.to(device)
    ours, ours_sc = causal_topk_with_scores(qd, kd, K)
    theirs = tr.row_blocked_topk(qd, kd, K)
    torch.cuda.synchronize()
    a = ours.long().sort(-1).values
    b = theirs.long().sort(-1).values
    diff_rows = (a != b).any(-1)                                   # (B, T)
    # rows t < K-1: valid keys {0..t} in both, so equal sets mean equal pad placement
    short = diff_rows[:, :K - 1]
    assert not short.any(), f"pad placement differs on rows {short.nonzero()[:8].tolist()}"
    full = diff_rows[:, K - 1:].nonzero().cpu()
    n_rows = B * (T - K + 1)
    _say(f"[crosscheck] {cfg}: {full.shape[0]} of {n_rows} full rows differ from torch "
         f"(pad rows: {B * (K - 1)} identical)")
    if full.shape[0] == 0:
        return
    qf, kf = qa.double(), ka.double()
    kmax = ka.float().abs().max().item()
    ours_c, theirs_c, sc_c = ours.cpu(), theirs.cpu(), ours_sc.cpu()
    worst = 0.0
    for bb, tt in full.tolist():
        t = tt + K - 1
        s_k = float(sc_c[bb, t, K - 1])                              # our K-th exact score
        eps = float(_near_tie_bound(qa[bb, t], kmax))
        sym = set(ours_c[bb, t].tolist()) ^ set(theirs_c[bb, t].tolist())
        for j in sym:
            assert 0 <= j <= t, f"non-causal index {j} in row {t}"
            s = float((qf[bb, t] * kf[bb, j]).sum())
            gap = abs(s - s_k)
            worst = max(worst, gap / eps)
            assert gap <= eps, f"{cfg} row {t}: key {j} differs by {gap:.3e} > {eps:.3e}"
    _say(f"[crosscheck] {cfg}: every difference is a near-tie (largest gap {worst:.3f} of the bound)")
    assert full.shape[0] <= max(16, n_rows // 200)


def test_topk_agrees_with_torch_on_fp32_distinct_scores(device):
    """Scores that are distinct and exact in fp32 in any summation order: q = (ints in
    [-3, 3], 1), k = (4096 x ints in [-30, 30], j), so s(t, j) = 4096 m + j with |m| < 2^12
    and every partial sum an integer below 2^24. No ties and no rounding: the index sets
    must equal torch's exactly on every row, pad rows included."""
    _say("[crosscheck] fp32 exact distinct scores")
    g = torch.Generator().manual_seed(41)
    B, T, R, K = 2, 3000, 32, 64
    qa = torch.randint(-3, 4, (B, T, R), generator=g).float()
    qa[..., -1] = 1.0
    ka = torch.randint(-30, 31, (B, T, R), generator=g).float() * 4096.0
    ka[..., -1] = torch.arange(T, dtype=torch.float32)
    qd, kd = qa.to(device), ka.to(device)
    ours = causal_topk(qd, kd, K).long().sort(-1).values
    theirs = tr.row_blocked_topk(qd, kd, K).long().sort(-1).values
    assert torch.equal(ours, theirs)
    assert torch.equal(ours.cpu(), native.causal_topk(qa, ka, K).long().sort(-1).values)
