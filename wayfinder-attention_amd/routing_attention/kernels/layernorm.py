"""Residual add + LayerNorm on the HIP kernel (wf_residual_layernorm_fwd).

Replaces, in the decoder's inference forward, the pair of PyTorch ops that the reference
block runs around each LayerNorm (routing_attention/models/transformer.py:50-73, final
norm :332): ``x = x + delta`` and ``F.layer_norm(x)``, in one pass that writes both the new
residual stream and its normalisation. Forward only: callers that need gradients keep the
PyTorch ops.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from routing_attention.kernels import _lib

MAX_WIDTH = 1024


def _rows_ok(t: torch.Tensor) -> bool:
    """(B, T, n) with a unit last stride, one row stride over all B * T rows, 16-byte rows."""
    es = t.element_size()
    return (t.dim() == 3 and t.stride(2) == 1 and t.data_ptr() % 16 == 0 and t.stride(1) * es % 16 == 0
            and (t.shape[0] == 1 or t.stride(0) == t.shape[1] * t.stride(1)))


def supported(x: torch.Tensor, ln: nn.LayerNorm, delta: torch.Tensor | None = None) -> bool:
    """Shapes and layouts the kernel takes, on a device where the library loads (anything
    else stays on the PyTorch ops: this pass only fuses ops PyTorch already provides)."""
    n = x.shape[-1]
    params = [p for p in (ln.weight, ln.bias) if p is not None]
    return (x.is_cuda and x.dtype in _lib.WF_DTYPE and _rows_ok(x) and n % 8 == 0 and n <= MAX_WIDTH
            and _lib.available()
            and tuple(ln.normalized_shape) == (n,)
            and (delta is None or (delta.shape == x.shape and delta.dtype == x.dtype and _rows_ok(delta)))
            and all(p.dtype == x.dtype and p.is_contiguous() and p.data_ptr() % 16 == 0 for p in params))


@torch.no_grad()
def residual_layer_norm(x: torch.Tensor, delta: torch.Tensor | None,
                        ln: nn.LayerNorm) -> tuple[torch.Tensor, torch.Tensor]:
    """(x + delta, ln(x + delta)) for x, delta (B, T, n); with delta None, (x, ln(x)).
    Rounds as the PyTorch ops do: the sum to x.dtype, the norm in fp32 rounded once."""
    _lib.require_device(x, *(t for t in (delta, ln.weight, ln.bias) if t is not None))
    B, T, n = x.shape
    y = torch.empty(B, T, n, dtype=x.dtype, device=x.device)
    s = torch.empty_like(y) if delta is not None else x
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.wf_residual_layernorm_fwd(
            x.data_ptr(), delta.data_ptr() if delta is not None else None, _lib.dtype_code(x),
            B * T, n, x.stride(1), delta.stride(1) if delta is not None else 0,
            ln.weight.data_ptr() if ln.weight is not None else None,
            ln.bias.data_ptr() if ln.bias is not None else None, float(ln.eps),
            s.data_ptr() if delta is not None else None, s.stride(1), y.data_ptr(), y.stride(1),
            _lib.stream_ptr(x.device))
    _lib.check(rc)
    return s, y
