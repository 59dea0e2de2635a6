"""GPU parity of the fused learned-address kernel (wf_address_project_fwd) against the
PyTorch ops it replaces (LearnedAddressModule.forward_query_key, reference
learned_address.py:39-46) and a float64 evaluation of the same formula."""

from __future__ import annotations

import sys

import pytest
import torch
import torch.nn.functional as F

from routing_attention.kernels.address import address_project
from routing_attention.models import LearnedAddressModule

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [
    # (B, T, d_model, R, dtype, similarity, normalize, x row padding)
    (2, 300, 256, 32, torch.bfloat16, "asymmetric", True, 0),
    (1, 65, 64, 16, torch.float32, "asymmetric", True, 0),
    (3, 100, 520, 32, torch.float16, "symmetric", True, 8),
    (1, 129, 264, 20, torch.bfloat16, "asymmetric", False, 16),
    (2, 64, 1024, 32, torch.float32, "symmetric", True, 0),
    # fewer tokens than one 16-token wave, spread over three batches (the MFMA kernel walks
    # a wave's tokens across batch boundaries)
    (3, 5, 64, 32, torch.bfloat16, "asymmetric", True, 0),
    (1, 7, 128, 12, torch.float16, "asymmetric", True, 8),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[4]}-d{c[2]}-R{c[3]}-{c[5]}-n{int(c[6])}" for c in CASES])
def test_address_kernel_vs_torch_ops(device, case):
    B, T, Dm, R, dtype, sim, norm, pad = case
    _say(f"[address] B{B} T{T} d{Dm} R{R} {dtype} {sim} normalize={norm}")
    torch.manual_seed(Dm + R)
    m = LearnedAddressModule(Dm, R, similarity=sim, normalize=norm).to(device=device, dtype=dtype)
    g = torch.Generator().manual_seed(T)
    base = torch.randn(B, T, Dm + pad, generator=g).to(dtype).to(device)
    x = base[..., :Dm]                      # strided rows when pad > 0
    kp = m.k_addr_proj
    with torch.no_grad():
        q, k = address_project(x, m.q_addr_proj.weight, m.q_addr_proj.bias,
                               kp.weight if kp is not None else None,
                               kp.bias if kp is not None else None, normalize=norm)
        # the PyTorch ops of the reference (forced by enabling grad on the input)
        xr = x.detach().clone().requires_grad_(True)
        with torch.enable_grad():
            tq, tk = m.forward_query_key(xr)
    torch.cuda.synchronize()
    assert q.shape == (B, T, R) and q.dtype == dtype
    if kp is None:
        assert k.data_ptr() == q.data_ptr()
    # float64 evaluation of the formula with the kernel's rounding steps
    def ref(w, b):
        y = x.double() @ w.double().T + b.double()
        if dtype != torch.float32:
            y = y.to(dtype).double()
        if norm:
            n = y.norm(dim=-1, keepdim=True)
            if dtype != torch.float32:
                n = n.to(dtype).double()
            y = y / n.clamp_min(1e-12)
        return y
    u = ULP[dtype]
    for got, tch, w, b in ((q, tq, m.q_addr_proj.weight, m.q_addr_proj.bias),
                           (k, tk, (kp or m.q_addr_proj).weight, (kp or m.q_addr_proj).bias)):
        r = ref(w, b)
        tch = tch.detach()
        if dtype == torch.float32:
            # fp32 accumulation over d_model products in another order: norm-wise 1e-5
            assert (got.double() - r).abs().max() <= 1e-5 * r.abs().max()
            assert (got - tch).abs().max() <= 1e-5 * tch.abs().max()
        else:
            # 16-bit: the roundings dominate -- within two units in the last place, and
            # equal to the PyTorch ops' result for all but a few percent of the elements
            assert ((got.double() - r).abs() <= 2 * u * r.abs().clamp_min(1e-3)).all()
            d = (got.float() - tch.float()).abs()
            assert (d <= 2 * u * tch.float().abs().clamp_min(1e-3)).all()
            assert (d > 0).float().mean() < 0.05


def test_module_uses_kernel_without_grad(device):
    """forward_query_key takes the kernel under no_grad and the PyTorch ops with grad."""
    _say("[address] module dispatch")
    import routing_attention.kernels.address as A

    m = LearnedAddressModule(128, 32).to(device)
    x = torch.randn(2, 50, 128, device=device)
    calls = []
    orig = A.address_project
    A.address_project = lambda *a, **k: calls.append(1) or orig(*a, **k)
    try:
        with torch.no_grad():
            q1, k1 = m.forward_query_key(x)
        q2, k2 = m.forward_query_key(x)
    finally:
        A.address_project = orig
    assert len(calls) == 1 and q2.requires_grad
    torch.testing.assert_close(q1, q2.detach(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(k1, k2.detach(), rtol=1e-5, atol=1e-6)
