"""Differentiable sparse readout on the HIP kernels (indices held fixed).

The reference trains through a gather formulation that autograd differentiates
(routing_attention/models/attention.py:35-55, _gather_kv_heads :58-69): it materialises
(B, H, T, K, D) copies of k and v and their gradients. Here the forward is
``wf_sparse_readout_fwd_lse`` (the readout plus the per-row base-2 log-sum-exp) and the
backward is ``wf_sparse_readout_bwd``: dq by a row pass, dk/dv by a key pass over the
transposed index lists, fp32 accumulation, deterministic. Indices get no gradient (as in
the reference, where they come out of a non-differentiable top-K).

Dropout on the attention weights (the reference's ``attn = dropout(softmax(...))``) runs
inside the same kernels (``wf_sparse_readout_fwd_dropout`` / ``_bwd_dropout``): the keep
mask is a hash of (seed, b, h, t, slot), recomputed by the backward instead of stored, and
the seed is drawn from torch's default generator, so ``torch.manual_seed`` makes a training
step reproducible. The mask is not torch's Bernoulli stream; its distribution is the same.
"""

from __future__ import annotations

import ctypes

import torch

from routing_attention.kernels import _lib


def _fast_layout(t: torch.Tensor) -> torch.Tensor:
    """The backward kernels read 16-byte rows with 32-bit offsets inside each (b, h) span:
    contiguous head dim and 16-byte aligned strides. Other layouts are copied once."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and t.shape[-1] % 8 == 0
          and all((s * es) % 16 == 0 for s in t.stride()[:-1]) and t.stride(2) >= 0)
    return t if ok else t.contiguous()


def _grad_like(t: torch.Tensor) -> torch.Tensor:
    # same memory layout as the input: (B, T, H, D) memory for the module's q/k/v views
    return torch.empty_like(t, memory_format=torch.preserve_format)


def readout_fwd_lse(q, k, v, indices, scale: float, flags: int = 0, dropout=None):
    """Forward readout and its (B, H, T) base-2 log-sum-exp (float32). ``dropout`` = (p, seed)
    drops attention weights with probability p (the log-sum-exp is that of all weights)."""
    B, H, T, D = q.shape
    K = indices.shape[-1]
    out = torch.empty_like(q, memory_format=torch.preserve_format)
    lse2 = torch.empty(B, H, T, dtype=torch.float32, device=q.device)
    lib = _lib.load()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(q), B, H, T, D,
            _lib.strides(q), _lib.strides(k), _lib.strides(v), indices.data_ptr(),
            _lib.strides(indices), K, float(scale), int(flags))
    with torch.cuda.device(q.device):
        if dropout is None:
            rc = lib.wf_sparse_readout_fwd_lse(*args, out.data_ptr(), _lib.strides(out),
                                               lse2.data_ptr(), _lib.stream_ptr(q.device))
        else:
            rc = lib.wf_sparse_readout_fwd_dropout(*args, float(dropout[0]), int(dropout[1]),
                                                   out.data_ptr(), _lib.strides(out),
                                                   lse2.data_ptr(), _lib.stream_ptr(q.device))
    _lib.check(rc)
    return out, lse2


def readout_bwd(q, k, v, indices, lse2, dout, scale: float, flags: int = 0, dropout=None):
    """(dq, dk, dv) of the readout for upstream gradient dout (``dropout`` as the forward's)."""
    q, k, v, dout = (_fast_layout(t) for t in (q, k, v, dout))
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    if indices.stride(-1) != 1:
        indices = indices.contiguous()
    B, H, T, D = q.shape
    K = indices.shape[-1]
    dq, dk, dv = _grad_like(q), _grad_like(k), _grad_like(v)
    lib = _lib.load()
    ws_bytes = lib.wf_sparse_readout_bwd_workspace_bytes(B, H, T, K)
    if ws_bytes == 0 and B * H * T * K > 0:
        raise _lib.WayfinderHipError(_lib.last_error())
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    a = _lib.ReadoutBwdArgs()
    a.q, a.k, a.v, a.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr()
    a.indices, a.lse2 = indices.data_ptr(), lse2.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    for name, t in (("q", q), ("k", k), ("v", v), ("dout", dout), ("dq", dq), ("dk", dk), ("dv", dv)):
        getattr(a, name + "_strides")[:] = list(t.stride())
    a.idx_strides[:] = list(indices.stride())
    a.B, a.H, a.T, a.D, a.K = B, H, T, D, K
    a.dtype, a.scale, a.flags = _lib.dtype_code(q), float(scale), int(flags)
    with torch.cuda.device(q.device):
        if dropout is None:
            rc = lib.wf_sparse_readout_bwd(ctypes.byref(a), _lib.stream_ptr(q.device))
        else:
            rc = lib.wf_sparse_readout_bwd_dropout(ctypes.byref(a), float(dropout[0]), int(dropout[1]),
                                                   _lib.stream_ptr(q.device))
    _lib.check(rc)
    return dq, dk, dv


class SparseReadoutFunction(torch.autograd.Function):
    """out = softmax_s(scale q.k_{idx_s}) v_{idx_s} per (b, h, t), differentiable in q, k, v."""

    @staticmethod
    def forward(ctx, q, k, v, indices, scale, flags, dropout):
        out, lse2 = readout_fwd_lse(q, k, v, indices, scale, flags, dropout)
        ctx.save_for_backward(q, k, v, indices, lse2)
        ctx.scale, ctx.flags, ctx.dropout = scale, flags, dropout
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, indices, lse2 = ctx.saved_tensors
        dq, dk, dv = readout_bwd(q, k, v, indices, lse2, dout, ctx.scale, ctx.flags, ctx.dropout)
        return dq, dk, dv, None, None, None, None


def draw_dropout_seed() -> int:
    """A 64-bit mask seed from torch's default (CPU) generator."""
    return int(torch.randint(0, 2 ** 63 - 1, (1,), dtype=torch.int64).item())


def sparse_readout(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor,
                   scale: float, *, mask_pads: bool = False, dropout_p: float = 0.0,
                   seed: int | None = None) -> torch.Tensor:
    """Differentiable sparse attention over shared (B, T, K) indices, (B, H, T, D) in q.dtype.

    Same result as ``sparse_meat_attention`` (reference fused_sparse.py:275-324 /
    attention.py:35-55); gradients flow to q, k and v. ``dropout_p`` > 0 drops attention
    weights after the softmax (each kept one scaled by 1 / (1 - p)), as the reference's
    non-fused training path does; ``seed`` fixes the mask (default: drawn from torch).
    """
    if not 0.0 <= float(dropout_p) <= 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {dropout_p}")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q/k/v must share a (B,H,T,D) shape: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v dtype mismatch: {q.dtype} {k.dtype} {v.dtype}")
    B, H, T, D = q.shape
    if indices.dim() != 3 or indices.shape[0] != B or indices.shape[1] != T:
        raise ValueError(f"indices must be (B,T,K)=({B},{T},K), got {tuple(indices.shape)}")
    if indices.shape[-1] == 0 or float(dropout_p) == 1.0:
        # softmax over an empty set sums to nothing, and dropout with p = 1 zeroes every
        # weight: a zero output, zero gradients
        return (q * 0.0 + k.sum() * 0.0 + v.sum() * 0.0) * 0.0
    _lib.require_device(q, k, v, indices)
    if indices.dtype != torch.int32:
        indices = indices.to(torch.int32)
    flags = _lib.WF_FLAG_MASK_PADS if mask_pads else 0
    dropout = None
    if float(dropout_p) > 0.0:
        dropout = (float(dropout_p), draw_dropout_seed() if seed is None else int(seed) & (2 ** 64 - 1))
    return SparseReadoutFunction.apply(q, k, v, indices, float(scale), flags, dropout)
