"""The fused forward's entry point that allocates nothing (wf_fused_topk_sparse_fwd_noalloc,
scratch in the library's own per-device array) against the entry point with a caller
workspace (wf_fused_topk_sparse_fwd), both through the C ABI: the same kernels run, so
indices and outputs must be bit-identical -- on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents)."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from routing_attention.kernels import _lib
from tests.helpers import addresses

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fill(qa, ka, q, k, v, K, out, idx, ws=None, ws_bytes=0):
    a = _lib.FusedArgs()
    a.q_search, a.k_search = qa.data_ptr(), ka.data_ptr()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.out_idx, a.out_scores = idx.data_ptr(), None
    a.workspace, a.workspace_bytes = (ws.data_ptr() if ws is not None else None), ws_bytes
    a.qs_strides[:] = list(qa.stride())
    a.ks_strides[:] = list(ka.stride())
    a.q_strides[:] = list(q.stride())
    a.k_strides[:] = list(k.stride())
    a.v_strides[:] = list(v.stride())
    a.out_strides[:] = list(out.stride())
    B, H, T, D = q.shape
    a.B, a.H, a.T, a.D, a.R, a.top_k = B, H, T, D, qa.shape[-1], K
    a.search_dtype = _lib.dtype_code(qa)
    a.dtype = _lib.dtype_code(q)
    a.scale = D ** -0.5
    a.flags = 0
    return a


def _inputs(B, H, T, D, R, seed, dtype, device):
    qa, ka = addresses(B, T, R, seed=seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 1)
    q, k, v = (torch.randn(B, T, H, D, generator=g).to(dtype).to(device).transpose(1, 2) for _ in range(3))
    return qa.to(device), ka.to(device), q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_entry_point_matches_workspace_entry_point(device, dtype):
    lib = _lib.load()
    stream = _lib.stream_ptr(device)
    for B, H, T, D, R, K, seed in [(2, 4, 3000, 64, 32, 128, 101), (1, 2, 500, 128, 32, 64, 102)]:
        _say(f"[noalloc] B{B} H{H} T{T} D{D} K{K} {dtype}")
        qa, ka, q, k, v = _inputs(B, H, T, D, R, seed, dtype, device)
        k_eff = min(K, T)
        out_ref = torch.empty(B, H, T, D, dtype=dtype, device=device)
        idx_ref = torch.empty(B, T, k_eff, dtype=torch.int32, device=device)
        ws_bytes = lib.wf_fused_workspace_bytes(B, T, R, K)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        a_ref = _fill(qa, ka, q, k, v, K, out_ref, idx_ref, ws, ws_bytes)
        _lib.check(lib.wf_fused_topk_sparse_fwd(ctypes.byref(a_ref), stream))
        out = torch.full((B, H, T, D), float("nan"), dtype=dtype, device=device)
        idx = torch.full((B, T, k_eff), -7, dtype=torch.int32, device=device)
        a = _fill(qa, ka, q, k, v, K, out, idx)      # no workspace: the library's scratch
        _lib.check(lib.wf_fused_topk_sparse_fwd_noalloc(ctypes.byref(a), stream))
        torch.cuda.synchronize()
        assert torch.equal(idx, idx_ref)
        bits = torch.int32 if dtype == torch.float32 else torch.int16   # bitwise comparison
        assert torch.equal(out.contiguous().view(bits), out_ref.contiguous().view(bits))


def test_noalloc_rejects_shapes_beyond_its_scratch(device):
    lib = _lib.load()
    limit = lib.wf_fused_noalloc_scratch_limit()
    assert limit == 1 << 20
    a = _lib.FusedArgs()
    a.B, a.H, a.T, a.D, a.R, a.top_k = 2048, 1, 65536, 64, 32, 128      # 2048 * 256 floats > 1 MiB
    rc = lib.wf_fused_topk_sparse_fwd_noalloc(ctypes.byref(a), None)
    assert rc == _lib.WF_ERR_UNSUPPORTED and "scratch" in _lib.last_error()
