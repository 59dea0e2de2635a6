"""ctypes binding of libwayfinder_hip.so (the C ABI in include/wayfinder_hip.h).

There is no other backend: a missing library or a missing ROCm device raises, it never
falls back to another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
LIB_PATH = os.environ.get(
    "WAYFINDER_HIP_LIB", os.path.join(_PKG_ROOT, "lib", "libwayfinder_hip.so")
)

WF_OK = 0
WF_ERR_INVALID_ARGUMENT = 1
WF_ERR_UNSUPPORTED = 2
WF_ERR_WORKSPACE = 3
WF_ERR_HIP = 4

WF_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
WF_FLAG_MASK_PADS = 0x1
WF_FLAG_SPLIT_PASS = 0x2
WF_FLAG_SINGLE_PASS = 0x4

# Exported symbols and their C signatures (kept in step with include/wayfinder_hip.h).
_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)


class FusedArgs(ctypes.Structure):
    _fields_ = [
        ("q_search", _p), ("k_search", _p), ("q", _p), ("k", _p), ("v", _p), ("out", _p),
        ("out_idx", _p), ("out_scores", _p), ("workspace", _p),
        ("workspace_bytes", ctypes.c_size_t),
        ("qs_strides", _i64 * 3), ("ks_strides", _i64 * 3),
        ("q_strides", _i64 * 4), ("k_strides", _i64 * 4), ("v_strides", _i64 * 4),
        ("out_strides", _i64 * 4),
        ("B", _i64), ("H", _i64), ("T", _i64), ("D", _i64), ("R", _i64), ("top_k", _i64),
        ("search_dtype", ctypes.c_int), ("dtype", ctypes.c_int),
        ("scale", ctypes.c_float), ("flags", ctypes.c_uint),
    ]


class ReadoutBwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", _p), ("k", _p), ("v", _p), ("dout", _p), ("indices", _p), ("lse2", _p),
        ("dq", _p), ("dk", _p), ("dv", _p), ("workspace", _p),
        ("workspace_bytes", ctypes.c_size_t),
        ("q_strides", _i64 * 4), ("k_strides", _i64 * 4), ("v_strides", _i64 * 4),
        ("dout_strides", _i64 * 4), ("dq_strides", _i64 * 4), ("dk_strides", _i64 * 4),
        ("dv_strides", _i64 * 4), ("idx_strides", _i64 * 3),
        ("B", _i64), ("H", _i64), ("T", _i64), ("D", _i64), ("K", _i64),
        ("dtype", ctypes.c_int), ("scale", ctypes.c_float), ("flags", ctypes.c_uint),
    ]


SIGNATURES = {
    "wf_abi_version": (ctypes.c_int, []),
    "wf_last_error": (ctypes.c_char_p, []),
    "wf_causal_topk_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "wf_causal_topk_fwd": (ctypes.c_int, [_p, _p, ctypes.c_int, _i64, _i64, _i64, _i64p, _i64p,
                                          _i64, _p, _p, _p, ctypes.c_size_t, _p]),
    "wf_sparse_readout_fwd": (ctypes.c_int, [_p, _p, _p, ctypes.c_int, _i64, _i64, _i64, _i64,
                                             _i64p, _i64p, _i64p, _p, _i64p, _i64,
                                             ctypes.c_float, ctypes.c_uint, _p, _i64p, _p]),
    "wf_sparse_readout_fwd_lse": (ctypes.c_int, [_p, _p, _p, ctypes.c_int, _i64, _i64, _i64, _i64,
                                                 _i64p, _i64p, _i64p, _p, _i64p, _i64,
                                                 ctypes.c_float, ctypes.c_uint, _p, _i64p, _p, _p]),
    "wf_sparse_readout_bwd_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "wf_sparse_readout_bwd": (ctypes.c_int, [ctypes.POINTER(ReadoutBwdArgs), _p]),
    "wf_sparse_readout_fwd_dropout": (ctypes.c_int, [_p, _p, _p, ctypes.c_int, _i64, _i64, _i64, _i64,
                                                     _i64p, _i64p, _i64p, _p, _i64p, _i64,
                                                     ctypes.c_float, ctypes.c_uint, ctypes.c_float,
                                                     ctypes.c_uint64, _p, _i64p, _p, _p]),
    "wf_sparse_readout_bwd_dropout": (ctypes.c_int, [ctypes.POINTER(ReadoutBwdArgs), ctypes.c_float,
                                                     ctypes.c_uint64, _p]),
    "wf_address_project_fwd": (ctypes.c_int, [_p, ctypes.c_int, _i64, _i64, _i64, _i64p, _p, _p,
                                              _p, _p, _i64, _i64, ctypes.c_int, _p, _i64p, _p,
                                              _i64p, _p]),
    "wf_residual_layernorm_fwd": (ctypes.c_int, [_p, _p, ctypes.c_int, _i64, _i64, _i64, _i64, _p, _p,
                                                 ctypes.c_float, _p, _i64, _p, _i64, _p]),
    "wf_fused_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "wf_fused_topk_sparse_fwd": (ctypes.c_int, [ctypes.POINTER(FusedArgs), _p]),
    "wf_fused_noalloc_scratch_limit": (ctypes.c_size_t, []),
    "wf_fused_topk_sparse_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(FusedArgs), _p]),
    "wf_probe_gather_sink_bytes": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "wf_probe_gather": (ctypes.c_int, [_p, _p, ctypes.c_int, _i64, _i64, _i64, _i64, _i64p, _i64p,
                                       _p, _i64p, _i64, _p, ctypes.c_size_t, _p]),
}

ABI_VERSION = 5

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class WayfinderHipError(RuntimeError):
    """A HIP runtime or launch failure inside libwayfinder_hip.so."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or has another ABI version."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libwayfinder_hip.so not found at {LIB_PATH}; build it with "
                "`python wayfinder-attention_amd/build.py` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.wf_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libwayfinder_hip.so ABI {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    """True when the library loads and a ROCm device is visible."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    try:
        load()
    except (OSError, RuntimeError):
        return False
    return True


def last_error() -> str:
    msg = load().wf_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    """Map a wf_status to the exception types the reference raises."""
    if rc == WF_OK:
        return
    msg = last_error()
    if rc in (WF_ERR_INVALID_ARGUMENT, WF_ERR_WORKSPACE):
        raise ValueError(msg)
    if rc == WF_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise WayfinderHipError(msg)


def strides(t: torch.Tensor):
    arr = (ctypes.c_int64 * t.dim())(*t.stride())
    return arr


def require_device(*tensors: torch.Tensor) -> None:
    """The HIP path runs on ROCm device tensors only: no host fallback exists."""
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "wayfinder-attention_amd runs on ROCm device tensors only; got a tensor on "
                f"{t.device}. Move inputs to the GPU (there is no CPU implementation)."
            )
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return WF_DTYPE[t.dtype]
    except KeyError:
        raise NotImplementedError(f"unsupported dtype {t.dtype}") from None


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
