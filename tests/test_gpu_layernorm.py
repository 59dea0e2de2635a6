"""GPU parity of the residual add + LayerNorm kernel (wf_residual_layernorm_fwd) against the
PyTorch ops it replaces in the decoder's inference forward (reference
routing_attention/models/transformer.py:50-73 and :332: x = x + delta, then nn.LayerNorm),
and of the decoder forward that uses it against the same forward on the PyTorch ops.

The sum is an elementwise add rounded once, as PyTorch's, so it must match exactly. The
norm's mean and variance are fp32 sums in another order than PyTorch's, so y matches to
fp32 accuracy before its rounding: within one unit in the last place of the storage type,
and exactly equal for all but a small fraction of the elements in 16-bit types."""

from __future__ import annotations

import sys

import pytest
import torch
import torch.nn as nn

from routing_attention.kernels.layernorm import residual_layer_norm, supported
from routing_attention.models import TransformerLM

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [
    # (B, T, n, dtype, delta, row padding, affine)
    (8, 2048, 256, torch.bfloat16, True, 0, True),      # the C2 decoder's shape
    (2, 300, 256, torch.bfloat16, False, 0, True),      # LayerNorm alone
    (1, 77, 1024, torch.float16, True, 16, True),       # widest row, strided rows
    (3, 50, 520, torch.float32, True, 0, True),         # n not a multiple of 128
    (2, 33, 64, torch.bfloat16, True, 8, False),        # no affine parameters
    (1, 5, 8, torch.float32, True, 0, True),            # narrowest row
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[3]}-n{c[2]}-d{int(c[4])}-pad{c[5]}" for c in CASES])
def test_residual_layernorm_matches_torch(device, case):
    B, T, n, dtype, with_delta, pad, affine = case
    _say(f"[layernorm] B{B} T{T} n{n} {dtype} delta={with_delta} pad={pad} affine={affine}")
    g = torch.Generator().manual_seed(n + T)
    base = (torch.randn(B, T, n + pad, generator=g) * 3 + 0.5).to(dtype).to(device)
    x = base[..., :n]
    delta = torch.randn(B, T, n, generator=g).to(dtype).to(device) if with_delta else None
    ln = nn.LayerNorm(n, elementwise_affine=affine).to(device=device, dtype=dtype)
    if affine:
        with torch.no_grad():
            ln.weight.copy_(torch.randn(n, generator=g).to(dtype))
            ln.bias.copy_(torch.randn(n, generator=g).to(dtype))
    assert supported(x, ln, delta)
    s, y = residual_layer_norm(x, delta, ln)
    torch.cuda.synchronize()
    with torch.no_grad():
        ts = x + delta if with_delta else x
        ty = ln(ts)
    assert torch.equal(s, ts)
    u = ULP[dtype]
    # one unit in the last place of the larger of |y| and 1 (the fp32 result before rounding
    # agrees with PyTorch's to ~1e-6 relative)
    bound = u * torch.maximum(ty.float().abs(), torch.ones_like(ty.float())) + 1e-5
    diff = (y.float() - ty.float()).abs()
    assert bool((diff <= bound).all()), f"max diff {diff.max().item():.3e}"
    if dtype != torch.float32:
        assert float((y != ty).float().mean()) < 0.02


def test_decoder_forward_with_fused_norms_matches_torch_ops(device):
    """The inference forward (fused add + norm passes) against the same model forced onto
    the per-block PyTorch ops (return_hidden_states takes the plain loop)."""
    _say("[layernorm] C2-like decoder: fused norms vs PyTorch ops")
    torch.manual_seed(2002)
    model = TransformerLM(128, 256, 2, 4, 1024, 1024, dropout=0.0, attention_type="learned_address",
                          routing_top_k=64, retrieval_config={"use_fused_sparse": True})
    model = model.eval().to(device=device, dtype=torch.bfloat16)
    ids = torch.randint(0, 128, (2, 1024), generator=torch.Generator().manual_seed(5)).to(device)
    with torch.no_grad():
        fast = model(ids)
        plain = model(ids, return_hidden_states=True)
    torch.cuda.synchronize()
    a, b = fast["logits"].float(), plain["logits"].float()
    rel = float((a - b).norm() / b.norm())
    # bf16 through 2 layers: one-ulp norm differences can move near-tie neighbours
    assert rel < 2e-2, rel
    assert abs(float(fast["loss"]) - float(plain["loss"])) < 2e-2 * float(plain["loss"])


def test_decoder_fp32_fused_norms_tight(device):
    _say("[layernorm] fp32 decoder: fused norms vs PyTorch ops")
    torch.manual_seed(7)
    model = TransformerLM(64, 128, 2, 2, 512, 256, dropout=0.0, attention_type="dense").eval().to(device)
    ids = torch.randint(0, 64, (2, 256), generator=torch.Generator().manual_seed(8)).to(device)
    with torch.no_grad():
        fast = model(ids)
        plain = model(ids, return_hidden_states=True)
    torch.cuda.synchronize()
    a, b = fast["logits"], plain["logits"]
    assert float((a - b).abs().max()) <= 1e-4 * float(b.abs().max())


def test_residual_layernorm_graph_replays(device):
    """Captured into a HIP graph and replayed several times, with eager work and host
    synchronisations in between: every replay equals the eager result."""
    _say("[layernorm] graph replays")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4, 512, 256, generator=g).to(torch.bfloat16).to(device)
    d = torch.randn(4, 512, 256, generator=g).to(torch.bfloat16).to(device)
    ln = nn.LayerNorm(256).to(device=device, dtype=torch.bfloat16)
    s_ref, y_ref = residual_layer_norm(x, d, ln)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        residual_layer_norm(x, d, ln)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s_g, y_g = residual_layer_norm(x, d, ln)
    for _ in range(4):
        s_g.zero_()
        y_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(s_g, s_ref) and torch.equal(y_g, y_ref)
        residual_layer_norm(x, d, ln)   # eager work between replays
        torch.cuda.synchronize()
