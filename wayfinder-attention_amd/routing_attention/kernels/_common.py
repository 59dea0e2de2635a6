"""Shared helpers (mirrors routing_attention/kernels/_common.py of the reference)."""

from __future__ import annotations

import torch

from routing_attention.kernels import _lib


def next_power_of_2(n: int) -> int:
    """Smallest power of two >= n (1 for n <= 1); reference _common.py:8-11."""
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def promote_compute_dtype(
    q: torch.Tensor,
    k: torch.Tensor,
    dtype: str | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.dtype]:
    """Retrieval input dtype (reference _common.py:14-31): an explicit dtype string wins,
    else fp16/bf16 inputs stay as they are and everything else becomes fp32. Scores are
    computed in fp32 from these values either way."""
    named = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
    if dtype in named:
        target = named[dtype]
    elif q.dtype in (torch.float16, torch.bfloat16):
        target = q.dtype
    else:
        target = torch.float32
    return q.to(target), k.to(target), target


def ensure_cuda_contiguous(*tensors: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """Reference _common.py:34-35 (kept for callers; the HIP path takes strides)."""
    return tuple(t.contiguous() if t.is_cuda else t for t in tensors)


def has_hip() -> bool:
    """True when libwayfinder_hip.so loads and a ROCm device is present (the role
    has_triton() plays in the reference, _common.py:38-46)."""
    return _lib.available()


# Reference name, same meaning on this build: "the fast kernels can run here".
has_triton = has_hip
