"""The streaming InfoNCE on the GPU (Phase-B address training without a (B, T, T)
similarity) against the reference's dense formulation in float64 on the CPU: loss value
and the gradients of the query and key addresses."""

from __future__ import annotations

import sys

import pytest
import torch

from routing_attention.losses import batched_infonce_loss
from tests.test_losses_cpu import _attention, _reference

pytestmark = pytest.mark.gpu


def test_streaming_infonce_on_device(device):
    print("[losses] streaming InfoNCE B2 T2048 R32 k32 fp32", flush=True)
    sys.stdout.flush()
    B, T, R, k = 2, 2048, 32, 32
    g = torch.Generator().manual_seed(11)
    q = torch.nn.functional.normalize(torch.randn(B, T, R, generator=g), dim=-1)
    kk = torch.nn.functional.normalize(torch.randn(B, T, R, generator=g), dim=-1)
    att = _attention(B, T, 12)
    qd, kd = q.to(device).requires_grad_(True), kk.to(device).requires_grad_(True)
    loss = batched_infonce_loss(qd, att.to(device), top_k=k, temperature=0.07, key_routing=kd)
    loss.backward()
    q64, k64 = q.double().requires_grad_(True), kk.double().requires_grad_(True)
    ref = _reference(q64, att.double(), k, 0.07, k64)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item())
    for a, b in ((qd.grad, q64.grad), (kd.grad, k64.grad)):
        err = (a.cpu().double() - b).abs().max() / b.abs().max()
        assert err < 1e-4, float(err)
