"""Fused sparse multi-head attention on MI355X (drop-in for the reference's
routing_attention/kernels/fused_sparse.py).

Pipeline: causal top-K on search vectors -> K/V gather -> softmax -> output, with the
indices shared across heads. Every method string runs the gfx950 kernels of
libwayfinder_hip.so; the (B, H, T, K, D) gathers the reference materialises never exist.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from routing_attention.kernels import _lib
from routing_attention.kernels._common import has_hip, next_power_of_2, promote_compute_dtype

_MAX_TRITON_K = 64
_MIN_TRITON_D = 16
_MAX_TRITON_D = 128


@dataclass
class SparseMeatConfig:
    """Launch options for the readout (reference fused_sparse.py:30-38).

    method / block_d / k_pad / num_warps / compute_dtype are accepted for compatibility;
    the HIP kernel picks its own tiling. This build's additions: ``mask_pads`` gives zero
    weight to the pad slots (s > t) of rows t < K-1 instead of attending them as the
    reference does; ``fused_pass`` selects how fused_sparse_attention runs -- "split"
    (retrieval kernel, then readout kernel), "single" (one kernel that retrieves each block
    of 16 query rows and reads them out for every head) or "auto" (the library's choice).
    """

    method: str = "auto"
    block_d: int | None = None
    k_pad: int | None = None
    num_warps: int = 4
    compute_dtype: str | None = None
    mask_pads: bool = False
    fused_pass: str = "auto"


def _resolve_sparse_meat_config(T: int, H: int, D: int, k_eff: int,
                                cfg: SparseMeatConfig | None) -> SparseMeatConfig:
    """Fill the derived fields (reference fused_sparse.py:41-57)."""
    cfg = cfg or SparseMeatConfig()
    return SparseMeatConfig(
        method=cfg.method,
        block_d=cfg.block_d or min(next_power_of_2(max(D, _MIN_TRITON_D)), _MAX_TRITON_D),
        k_pad=cfg.k_pad or min(next_power_of_2(max(k_eff, 1)), _MAX_TRITON_K),
        num_warps=cfg.num_warps,
        compute_dtype=cfg.compute_dtype,
        mask_pads=cfg.mask_pads,
        fused_pass=cfg.fused_pass,
    )


def fused_sparse_attention_available() -> bool:
    """True when the HIP kernels can run (reference fused_sparse.py:60-61)."""
    return has_hip()


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if q.dim() != 4:
        raise ValueError(f"expected q of shape (B,H,T,D), got {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q/k/v shape mismatch: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v dtype mismatch: {q.dtype} {k.dtype} {v.dtype}")


_PASS_FLAGS = {"auto": 0, "split": _lib.WF_FLAG_SPLIT_PASS, "single": _lib.WF_FLAG_SINGLE_PASS}


def _flags(cfg: SparseMeatConfig | None) -> int:
    if cfg is None:
        return 0
    if cfg.fused_pass not in _PASS_FLAGS:
        raise ValueError(f"fused_pass must be one of {sorted(_PASS_FLAGS)}, got {cfg.fused_pass!r}")
    return (_lib.WF_FLAG_MASK_PADS if cfg.mask_pads else 0) | _PASS_FLAGS[cfg.fused_pass]


@torch.no_grad()
def sparse_meat_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    indices: torch.Tensor,
    scale: float,
    *,
    method: str = "auto",
    config: SparseMeatConfig | None = None,
) -> torch.Tensor:
    """Multi-head sparse attention on pre-selected neighbours (reference
    fused_sparse.py:275-324).

    Args:
        q, k, v: (B, H, T, D) on a ROCm device, same dtype (fp32 / fp16 / bf16), any strides.
        indices: (B, T, K) neighbour positions shared across heads (cast to int32).
        scale: multiplies q.k before the softmax.
    Returns:
        (B, H, T, D) in q.dtype: softmax over the K slots, fp32 accumulation.
    """
    del method
    _check_qkv(q, k, v)
    if indices.dtype != torch.int32:
        indices = indices.to(torch.int32)
    B, H, T, D = q.shape
    if indices.dim() != 3 or indices.shape[0] != B or indices.shape[1] != T:
        raise ValueError(f"indices must be (B,T,K)=({B},{T},K), got {tuple(indices.shape)}")
    K = indices.shape[-1]
    out = torch.empty(B, H, T, D, dtype=q.dtype, device=q.device)
    if K == 0:
        return out.zero_()   # softmax over an empty set sums to nothing, as in the reference
    _lib.require_device(q, k, v, indices)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.wf_sparse_readout_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(q), B, H, T, D,
            _lib.strides(q), _lib.strides(k), _lib.strides(v),
            indices.data_ptr(), _lib.strides(indices), K, float(scale), _flags(config),
            out.data_ptr(), _lib.strides(out), _lib.stream_ptr(q.device),
        )
    _lib.check(rc)
    return out


def _fused(q_search, k_search, q, k, v, top_k, scale, cfg, out: torch.Tensor):
    """One wf_fused_topk_sparse_fwd call writing into ``out`` (any (B,H,T,D) strides)."""
    B, H, T, D = q.shape
    R = q_search.shape[-1]
    k_eff = min(int(top_k), T)
    dev = q.device
    idx = torch.empty(B, T, k_eff, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws_bytes = lib.wf_fused_workspace_bytes(B, T, R, int(top_k))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    a = _lib.FusedArgs()
    a.q_search, a.k_search = q_search.data_ptr(), k_search.data_ptr()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.out_idx, a.out_scores = idx.data_ptr(), None
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    a.qs_strides[:] = list(q_search.stride())
    a.ks_strides[:] = list(k_search.stride())
    a.q_strides[:] = list(q.stride())
    a.k_strides[:] = list(k.stride())
    a.v_strides[:] = list(v.stride())
    a.out_strides[:] = list(out.stride())
    a.B, a.H, a.T, a.D, a.R, a.top_k = B, H, T, D, R, int(top_k)
    a.search_dtype = _lib.dtype_code(q_search)
    a.dtype = _lib.dtype_code(q)
    a.scale = float(scale)
    a.flags = _flags(cfg)
    with torch.cuda.device(dev):
        rc = lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), _lib.stream_ptr(dev))
    _lib.check(rc)
    return idx


def _prepare_fused(q_search, k_search, q, k, v, top_k):
    if q_search.shape != k_search.shape:
        raise ValueError(f"query/key shape mismatch: {q_search.shape} vs {k_search.shape}")
    if q_search.dim() != 3:
        raise ValueError(f"expected (B,T,R), got {tuple(q_search.shape)}")
    _check_qkv(q, k, v)
    B, H, T, D = q.shape
    if q_search.shape[0] != B or q_search.shape[1] != T:
        raise ValueError(f"search vectors {tuple(q_search.shape)} do not match q {tuple(q.shape)}")
    qs, ks, _ = promote_compute_dtype(q_search, k_search, None)
    _lib.require_device(qs, ks, q, k, v)
    return qs, ks


@torch.no_grad()
def fused_sparse_attention(
    q_search: torch.Tensor,
    k_search: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    top_k: int,
    scale: float,
    *,
    retrieval_method: str = "auto",
    meat_method: str = "auto",
    meat_config: SparseMeatConfig | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Causal top-K retrieval + sparse attention (reference fused_sparse.py:327-356).

    Args:
        q_search, k_search: (B, T, R) search-space vectors.
        q, k, v: (B, H, T, D) projections (any strides).
    Returns:
        out (B, H, T, D) in q.dtype, indices (B, T, k_eff) int32.
    """
    del retrieval_method, meat_method
    qs, ks = _prepare_fused(q_search, k_search, q, k, v, top_k)
    B, H, T, D = q.shape
    out = torch.empty(B, H, T, D, dtype=q.dtype, device=q.device)
    if min(int(top_k), T) <= 0:
        return out.zero_(), torch.zeros(B, T, 0, dtype=torch.int32, device=q.device)
    idx = _fused(qs, ks, q, k, v, top_k, scale, meat_config, out)
    return out, idx


@torch.no_grad()
def fused_sparse_attention_bthd(
    q_search: torch.Tensor,
    k_search: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    top_k: int,
    scale: float,
    *,
    meat_config: SparseMeatConfig | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fused_sparse_attention with the output laid out as (B, T, H, D) in memory, which
    is what the attention module flattens next; saves the transpose copy. Not in the
    reference API."""
    qs, ks = _prepare_fused(q_search, k_search, q, k, v, top_k)
    B, H, T, D = q.shape
    out_bthd = torch.empty(B, T, H, D, dtype=q.dtype, device=q.device)
    if min(int(top_k), T) <= 0:
        return out_bthd.zero_(), torch.zeros(B, T, 0, dtype=torch.int32, device=q.device)
    idx = _fused(qs, ks, q, k, v, top_k, scale, meat_config, out_bthd.transpose(1, 2))
    return out_bthd, idx
