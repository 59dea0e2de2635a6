"""ctypes binding of the C oracle ``libwf_oracle.so`` (test infrastructure only).

Semantics are documented in ``wf_oracle.c``; every function here converts its tensor
arguments to contiguous CPU fp32 (exact for bf16/fp16 inputs) before calling into C.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwf_oracle.so")
_lib = None

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def build() -> None:
    """Compile libwf_oracle.so from wf_oracle.c (gcc, via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        l.wfo_score.restype = ctypes.c_float
        l.wfo_score.argtypes = [_ptr, _ptr, _i64]
        l.wfo_causal_topk_rows.restype = None
        l.wfo_causal_topk_rows.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                                           _i64, _ptr, _ptr]
        l.wfo_causal_topk_rowlist.restype = None
        l.wfo_causal_topk_rowlist.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64,
                                              _ptr, _ptr]
        l.wfo_causal_topk.restype = None
        l.wfo_causal_topk.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _ptr]
        l.wfo_sparse_readout.restype = None
        l.wfo_sparse_readout.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                                         _i64, ctypes.c_float, ctypes.c_uint, _ptr]
        l.wfo_sparse_readout_dropout.restype = None
        l.wfo_sparse_readout_dropout.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                                                 _i64, ctypes.c_float, ctypes.c_uint,
                                                 ctypes.c_float, ctypes.c_uint64, _ptr]
        l.wfo_dropout_mask.restype = None
        l.wfo_dropout_mask.argtypes = [_i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_uint64, _ptr]
        l.wfo_sparse_readout_rows.restype = None
        l.wfo_sparse_readout_rows.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                                              _i64, _ptr, _i64, ctypes.c_float, ctypes.c_uint,
                                              _ptr]
        _lib = l
    return _lib


def _f32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().to("cpu", torch.float32).contiguous().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def score(q_row, k_row) -> float:
    """fp32 FMA-chain score of one (query, key) pair."""
    q = _f32(q_row).ravel()
    k = _f32(k_row).ravel()
    return float(lib().wfo_score(_p(q), _p(k), q.size))


def causal_topk(query, key, top_k: int, *, return_scores: bool = False):
    """(B,T,R) x2 -> int32 (B,T,k_eff) canonical indices (+ fp32 scores)."""
    q = _f32(query)
    k = _f32(key)
    B, T, R = q.shape
    k_eff = min(int(top_k), T)
    idx = np.empty((B, T, k_eff), dtype=np.int32)
    sc = np.empty((B, T, k_eff), dtype=np.float32)
    if k_eff > 0:
        lib().wfo_causal_topk(_p(q), _p(k), B, T, R, int(top_k), _p(idx), _p(sc))
    idx_t = torch.from_numpy(idx)
    return (idx_t, torch.from_numpy(sc)) if return_scores else idx_t


def causal_topk_rows(query, key, top_k: int, b: int, row0: int, row1: int,
                     *, return_scores: bool = False):
    """Rows [row0, row1) of batch b only (cheap spot checks at full T)."""
    q = _f32(query)
    k = _f32(key)
    B, T, R = q.shape
    k_eff = min(int(top_k), T)
    n = row1 - row0
    idx = np.empty((n, k_eff), dtype=np.int32)
    sc = np.empty((n, k_eff), dtype=np.float32)
    if k_eff > 0 and n > 0:
        lib().wfo_causal_topk_rows(_p(q), _p(k), B, T, R, int(top_k), b, row0, row1,
                                   _p(idx), _p(sc))
    idx_t = torch.from_numpy(idx)
    return (idx_t, torch.from_numpy(sc)) if return_scores else idx_t


def causal_topk_rowlist(query, key, top_k: int, rows_bt, *, return_scores: bool = False):
    """Selected (b, t) rows, rows_bt (n, 2) int: (n, k_eff) canonical indices (+ scores)."""
    q = _f32(query)
    k = _f32(key)
    B, T, R = q.shape
    k_eff = min(int(top_k), T)
    rb = np.ascontiguousarray(torch.as_tensor(rows_bt).to(torch.int64).numpy(), dtype=np.int64)
    n = rb.shape[0]
    idx = np.empty((n, k_eff), dtype=np.int32)
    sc = np.empty((n, k_eff), dtype=np.float32)
    if k_eff > 0 and n > 0:
        lib().wfo_causal_topk_rowlist(_p(q), _p(k), B, T, R, int(top_k), _p(rb), n, _p(idx), _p(sc))
    idx_t = torch.from_numpy(idx)
    return (idx_t, torch.from_numpy(sc)) if return_scores else idx_t


def sparse_readout(q, k, v, indices, scale: float, flags: int = 0) -> torch.Tensor:
    """(B,H,T,D) x3 + int32 (B,T,K) -> float64 (B,H,T,D)."""
    qn, kn, vn = _f32(q), _f32(k), _f32(v)
    B, H, T, D = qn.shape
    idx = np.ascontiguousarray(
        indices.detach().cpu().to(torch.int32).numpy() if isinstance(indices, torch.Tensor)
        else indices, dtype=np.int32)
    K = idx.shape[-1]
    out = np.empty((B, H, T, D), dtype=np.float64)
    lib().wfo_sparse_readout(_p(qn), _p(kn), _p(vn), B, H, T, D, _p(idx), K,
                             float(scale), int(flags), _p(out))
    return torch.from_numpy(out)


def sparse_readout_dropout(q, k, v, indices, scale: float, dropout_p: float, seed: int,
                           flags: int = 0) -> torch.Tensor:
    """The readout with dropout on the attention weights (hash mask of seed), float64."""
    qn, kn, vn = _f32(q), _f32(k), _f32(v)
    B, H, T, D = qn.shape
    idx = np.ascontiguousarray(indices.detach().cpu().to(torch.int32).numpy(), dtype=np.int32)
    K = idx.shape[-1]
    out = np.empty((B, H, T, D), dtype=np.float64)
    lib().wfo_sparse_readout_dropout(_p(qn), _p(kn), _p(vn), B, H, T, D, _p(idx), K, float(scale),
                                     int(flags), float(dropout_p), int(seed) & (2 ** 64 - 1), _p(out))
    return torch.from_numpy(out)


def dropout_mask(B: int, H: int, T: int, K: int, dropout_p: float, seed: int) -> torch.Tensor:
    """(B, H, T, K) bool keep mask of the readout's dropout for this seed."""
    out = np.empty((B, H, T, K), dtype=np.uint8)
    lib().wfo_dropout_mask(B, H, T, K, float(dropout_p), int(seed) & (2 ** 64 - 1), _p(out))
    return torch.from_numpy(out).bool()


def sparse_readout_rows(q, k, v, rows_bt, indices, scale: float, flags: int = 0) -> torch.Tensor:
    """Readout of selected (b, t) rows only: rows_bt (n, 2) int, indices (n, K) int32 (the
    index row of each pair) -> float64 (n, H, D). q, k, v (B,H,T,D) as in sparse_readout."""
    qn, kn, vn = _f32(q), _f32(k), _f32(v)
    B, H, T, D = qn.shape
    rb = np.ascontiguousarray(torch.as_tensor(rows_bt).to(torch.int64).numpy(), dtype=np.int64)
    idx = np.ascontiguousarray(torch.as_tensor(indices).cpu().to(torch.int32).numpy(), dtype=np.int32)
    n, K = idx.shape
    assert rb.shape == (n, 2)
    out = np.empty((n, H, D), dtype=np.float64)
    if n > 0:
        lib().wfo_sparse_readout_rows(_p(qn), _p(kn), _p(vn), B, H, T, D, _p(rb), n, _p(idx), K,
                                      float(scale), int(flags), _p(out))
    return torch.from_numpy(out)


def fused(q_search, k_search, q, k, v, top_k: int, scale: float, flags: int = 0):
    """causal_topk then sparse_readout; returns (float64 out, int32 indices)."""
    idx = causal_topk(q_search, k_search, top_k)
    return sparse_readout(q, k, v, idx, scale, flags), idx


def pad_index(t: int, s: int, k_eff: int, T: int) -> int:
    """Pad index of slot s of row t (causal_topk.py:53-56)."""
    return (t + k_eff + s + 1) % T
