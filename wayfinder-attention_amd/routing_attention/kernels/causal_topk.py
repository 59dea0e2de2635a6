"""Causal top-K inner-product retrieval on MI355X (drop-in for the reference's
routing_attention/kernels/causal_topk.py).

Every method string the reference accepts runs the same gfx950 kernel
(``wf_causal_topk_fwd`` in libwayfinder_hip.so): an MFMA-screened streaming top-K that
never writes scores to HBM and selects on exact fp32 scores (FMA chain over the address
dims in ascending order), ties to the lower key index. The result set equals the
reference's for every row; the slot order is canonical (score descending, pads last)
where the reference's is unspecified (torch.topk(sorted=False)).
"""

from __future__ import annotations

import torch

from routing_attention.kernels import _lib
from routing_attention.kernels._common import has_hip, promote_compute_dtype

# Method names of the reference (causal_topk.py:480-487, 501-521). All map to the HIP kernel.
METHODS = ("auto", "fused_causal", "triton", "tiled", "streaming", "brute_force")

# Largest address dim (R) and k_eff the HIP kernel takes (include/wayfinder_hip.h).
MAX_ADDRESS_DIM = 256
MAX_TOP_K = 512


def causal_topk_available() -> bool:
    """True when the HIP kernels can run (reference causal_topk.py:33-34)."""
    return has_hip()


def _check_shapes(query: torch.Tensor, key: torch.Tensor) -> None:
    # reference causal_topk.py:489-492
    if query.shape != key.shape:
        raise ValueError(f"query/key shape mismatch: {query.shape} vs {key.shape}")
    if query.dim() != 3:
        raise ValueError(f"expected (B,T,R), got {tuple(query.shape)}")


def _run_topk(q: torch.Tensor, k: torch.Tensor, top_k: int, want_scores: bool):
    _lib.require_device(q, k)
    lib = _lib.load()
    B, T, R = q.shape
    k_eff = min(int(top_k), T)
    dev = q.device
    out_idx = torch.empty(B, T, k_eff, dtype=torch.int32, device=dev)
    out_sc = torch.empty(B, T, k_eff, dtype=torch.float32, device=dev) if want_scores else None
    ws_bytes = lib.wf_causal_topk_workspace_bytes(B, T, R, int(top_k))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.wf_causal_topk_fwd(
            q.data_ptr(), k.data_ptr(), _lib.dtype_code(q), B, T, R,
            _lib.strides(q), _lib.strides(k), int(top_k), out_idx.data_ptr(),
            out_sc.data_ptr() if out_sc is not None else None,
            ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev),
        )
    _lib.check(rc)
    return out_idx, out_sc


@torch.no_grad()
def causal_topk(
    query: torch.Tensor,
    key: torch.Tensor,
    top_k: int,
    *,
    method: str = "auto",
    dtype: str | None = None,
    prefer_triton: bool = False,
) -> torch.Tensor:
    """Causal top-K retrieval (reference causal_topk.py:470-521).

    Args:
        query, key: (B, T, R) address vectors on a ROCm device.
        top_k: neighbours per query; k_eff = min(top_k, T).
        method: any reference method name; all run the HIP kernel.
        dtype: optional "float16" | "bfloat16" | "float32" cast applied before scoring
            (scores are fp32 of the cast values, as in the reference).
        prefer_triton: accepted for signature compatibility; no effect.
    Returns:
        int32 (B, T, k_eff). Row t holds its k_eff best keys j <= t; rows with t+1 < k_eff
        hold pad index (t + k_eff + s + 1) % T in slots s > t, as the reference does.
    """
    del method, prefer_triton
    _check_shapes(query, key)
    B, T, _ = query.shape
    k_eff = min(int(top_k), T)
    if k_eff <= 0:
        return torch.zeros(B, T, 0, dtype=torch.int32, device=query.device)
    q, k, _ = promote_compute_dtype(query, key, dtype)
    idx, _ = _run_topk(q, k, top_k, want_scores=False)
    return idx


@torch.no_grad()
def causal_topk_with_scores(
    query: torch.Tensor,
    key: torch.Tensor,
    top_k: int,
    *,
    dtype: str | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """causal_topk plus the fp32 score of every slot (-inf in pad slots). Not in the
    reference API; used to check the selection against recomputed scores."""
    _check_shapes(query, key)
    B, T, _ = query.shape
    k_eff = min(int(top_k), T)
    if k_eff <= 0:
        z = torch.zeros(B, T, 0, dtype=torch.int32, device=query.device)
        return z, z.float()
    q, k, _ = promote_compute_dtype(query, key, dtype)
    return _run_topk(q, k, top_k, want_scores=True)


@torch.no_grad()
def causal_topk_reference(query: torch.Tensor, key: torch.Tensor, top_k: int) -> torch.Tensor:
    """Exact causal top-K in descending score order (reference causal_topk.py:60-72, the
    brute-force baseline). Computed by the same HIP kernel, which already emits sorted
    order; slots without a causal key carry the reference's pad indices instead of
    whatever torch.topk leaves in its -inf slots."""
    _check_shapes(query, key)
    B, T, _ = query.shape
    k_eff = min(int(top_k), T)
    if k_eff <= 0:
        return torch.zeros(B, T, 0, dtype=torch.int32, device=query.device)
    idx, _ = _run_topk(query.float(), key.float(), top_k, want_scores=False)
    return idx
