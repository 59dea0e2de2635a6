"""Learned-address projection + L2 normalisation on the HIP kernel (wf_address_project_fwd).

Replaces the two Linear layers and F.normalize calls of
LearnedAddressModule.forward_query_key (reference learned_address.py:39-46) with one pass
over the hidden states, rounding as those PyTorch ops do. Forward only: callers that need
gradients through the addresses keep the PyTorch ops.
"""

from __future__ import annotations

import torch

from routing_attention.kernels import _lib

MAX_ADDRESS_DIM = 32


def supported(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor | None) -> bool:
    """Shapes and layouts the kernel takes (anything else stays on the PyTorch ops)."""
    ws = [w for w in (wq, wk) if w is not None]
    es = x.element_size()
    return (x.is_cuda and x.dim() == 3 and x.dtype in _lib.WF_DTYPE and x.shape[-1] % 8 == 0
            and wq.shape[0] <= MAX_ADDRESS_DIM and x.stride(-1) == 1 and x.data_ptr() % 16 == 0
            and all(s * es % 16 == 0 for s in x.stride()[:2])
            and all(w.dtype == x.dtype and w.stride(-1) == 1 and w.data_ptr() % 16 == 0
                    and w.stride(0) * es % 16 == 0 for w in ws))


@torch.no_grad()
def address_project(x: torch.Tensor, wq: torch.Tensor, bq: torch.Tensor | None,
                    wk: torch.Tensor | None, bk: torch.Tensor | None,
                    normalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """x (B, T, d_model) -> (q, k), each (B, T, R) in x.dtype; k is q when wk is None."""
    B, T, Dm = x.shape
    R = wq.shape[0]
    if wk is not None and wk.shape != wq.shape:
        raise ValueError(f"query/key projections differ: {tuple(wq.shape)} vs {tuple(wk.shape)}")
    for w in (wq, wk):
        if w is not None and w.shape[1] != Dm:
            raise ValueError(f"projection {tuple(w.shape)} does not take d_model={Dm}")
    _lib.require_device(x, wq)
    q = torch.empty(B, T, R, dtype=x.dtype, device=x.device)
    k = torch.empty_like(q) if wk is not None else q
    lib = _lib.load()
    bq = bq.to(x.dtype) if bq is not None else None
    bk = bk.to(x.dtype) if bk is not None else None
    with torch.cuda.device(x.device):
        rc = lib.wf_address_project_fwd(
            x.data_ptr(), _lib.dtype_code(x), B, T, Dm, _lib.strides(x), wq.data_ptr(),
            bq.data_ptr() if bq is not None else None,
            wk.data_ptr() if wk is not None else None,
            bk.data_ptr() if bk is not None else None,
            wq.stride(0), R, int(bool(normalize)), q.data_ptr(), _lib.strides(q),
            k.data_ptr() if wk is not None else None, _lib.strides(k) if wk is not None else None,
            _lib.stream_ptr(x.device))
    _lib.check(rc)
    return q, k
