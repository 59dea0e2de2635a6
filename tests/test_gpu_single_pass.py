"""GPU parity of the single-pass fused kernel (wf_fused_topk_sparse_fwd with
WF_FLAG_SINGLE_PASS: each workgroup retrieves 16 query rows and reads them out for every
head in the same kernel) against the C oracle and against the split path (retrieval kernel,
then readout kernel): indices bit-exact, outputs within the dtype's tolerance of the oracle.
Covers both template shapes of its readout stage (D / 8 lanes per head, one or two wave
loads per neighbour), ragged T, K below 128 and up to 256, pad masking and the contiguous
(B, H, T, D) layout next to the module's (B, T, H, D) memory."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import native
from routing_attention.kernels import SparseMeatConfig, fused_sparse_attention
from tests.helpers import addresses, plant, rel_err

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(B, H, T, D, R, seed, dist="normal", layout="bthd", ka_fn=None):
    qa, ka = addresses(B, T, R, seed=seed, dtype=torch.float32, dist=dist)
    if ka_fn is not None:
        ka = ka_fn(qa, ka)
    qa, ka = qa.to(torch.bfloat16), ka.to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 1)
    if layout == "bthd":
        q, k, v = (torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).transpose(1, 2) for _ in range(3))
    else:
        q, k, v = (torch.randn(B, H, T, D, generator=g).to(torch.bfloat16) for _ in range(3))
    return qa, ka, q, k, v


def _run(device, qa, ka, q, k, v, K, mode, mask_pads=False):
    cfg = SparseMeatConfig(fused_pass=mode, mask_pads=mask_pads)
    out, idx = fused_sparse_attention(qa.to(device), ka.to(device), q.to(device), k.to(device),
                                      v.to(device), K, q.shape[-1] ** -0.5, meat_config=cfg)
    torch.cuda.synchronize()
    return out, idx


CASES = [
    # B, H, T, D, K, layout, note
    (1, 8, 16384, 64, 128, "bthd", "config 4"),
    (2, 8, 1000, 64, 100, "bthd", "ragged T, K=100"),
    (1, 4, 777, 128, 128, "bthd", "D=128, 16 lanes per head, one load per neighbour"),
    (1, 16, 600, 64, 200, "bthd", "H=16, two loads per neighbour, K=200"),
    (2, 8, 900, 128, 256, "bhtd", "D=128 H=8 K=256, contiguous (B,H,T,D)"),
]


@pytest.mark.parametrize("B,H,T,D,K,layout,note", CASES)
def test_single_pass_matches_oracle_and_split(device, B, H, T, D, K, layout, note):
    _say(f"[single-pass] B{B} H{H} T{T} D{D} K{K} {layout} ({note})")
    qa, ka, q, k, v = _inputs(B, H, T, D, 32, seed=B * 7 + H * 131 + T + K, layout=layout)
    out1, idx1 = _run(device, qa, ka, q, k, v, K, "single")
    out2, idx2 = _run(device, qa, ka, q, k, v, K, "split")
    ref_idx = native.causal_topk(qa, ka, K)
    assert torch.equal(idx1.cpu(), ref_idx)
    assert torch.equal(idx2.cpu(), ref_idx)
    ref = native.sparse_readout(q, k, v, ref_idx, D ** -0.5)
    e1, e2 = rel_err(out1.float(), ref), rel_err(out2.float(), ref)
    _say(f"[single-pass] rel err single {e1:.2e} split {e2:.2e}")
    assert e1 < 2e-2 and e2 < 2e-2


def test_single_pass_config3_planted_and_mask_pads(device):
    _say("[single-pass] config 3 planted, mask_pads")
    B, H, T, D, K = 4, 8, 4096, 64, 128
    qa, ka, q, k, v = _inputs(B, H, T, D, 32, seed=1003, ka_fn=lambda a, b: plant(a, b, 0.01, seed=2003)[0])
    out, idx = _run(device, qa, ka, q, k, v, K, "single", mask_pads=True)
    ref_idx = native.causal_topk(qa, ka, K)
    assert torch.equal(idx.cpu(), ref_idx)
    ref = native.sparse_readout(q, k, v, ref_idx, D ** -0.5, flags=1)
    assert rel_err(out.float(), ref) < 2e-2
    # row 0 with masked pads attends to key 0 only
    assert torch.allclose(out[:, :, 0].float().cpu(), v[:, :, 0].float(), atol=1e-2)


def test_single_pass_config5_sampled(device):
    """Config 5 shape (T=65536, D=128, K=256, Student-t) on the single-pass kernel."""
    B, H, T, D, K = 1, 8, 65536, 128, 256
    _say(f"[single-pass] config 5: B{B} H{H} T{T} D{D} K{K}")
    qa, ka, q, k, v = _inputs(B, H, T, D, 32, seed=1005, dist="student_t")
    out, idx = _run(device, qa, ka, q, k, v, K, "single")
    g = torch.Generator().manual_seed(3006)
    ts = torch.cat([torch.arange(260), (torch.randperm(T - 324, generator=g)[:700] + 260).sort().values,
                    torch.arange(T - 64, T)])
    rows = torch.stack([torch.zeros_like(ts), ts], dim=1)
    ref_idx = native.causal_topk_rowlist(qa, ka, K, rows)
    assert torch.equal(idx.cpu()[0, ts], ref_idx)
    ref = native.sparse_readout_rows(q, k, v, rows, ref_idx, D ** -0.5)
    got = out.cpu()[0, :, ts].transpose(0, 1).float()
    assert rel_err(got, ref) < 2e-2


def test_single_pass_rejects_unsupported_layouts(device):
    qa, ka, q, k, v = _inputs(1, 2, 300, 32, 32, seed=5)      # H * D = 64: not a single-pass shape
    with pytest.raises(NotImplementedError, match="single-pass"):
        _run(device, qa, ka, q, k, v, 128, "single")
    out, idx = _run(device, qa, ka, q, k, v, 128, "auto")       # auto falls back to the split path
    assert torch.equal(idx.cpu(), native.causal_topk(qa, ka, 128))
