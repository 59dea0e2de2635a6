"""Retrieval configuration (mirrors routing_attention/retrieval/index.py of the reference
for the fields and the retriever entry the hot path needs).

``RetrievalConfig.use_fused_sparse`` and ``method`` route LearnedAddressSparseAttention
onto the fused path (reference index.py:82-98, attention.py:31-32). ``RoutingRetriever``
keeps only the exact causal retrieval; every method name runs the HIP causal_topk kernel
(FAISS/HNSW indexes are not part of this build).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
import torch.nn as nn

from routing_attention.kernels.causal_topk import causal_topk

RetrievalMethod = Literal["fused_causal", "brute_force", "faiss_flat", "faiss_hnsw", "auto"]


@dataclass
class RetrievalConfig:
    """Reference index.py:82-98 (same fields and defaults)."""

    method: RetrievalMethod = "auto"
    top_k: int = 32
    max_seq_len: int = 8192
    oversample: int = 4
    dtype: Literal["float32", "float16", "bfloat16"] = "float16"
    brute_force_max_seq: int = 2048
    faiss_flat_max_seq: int = 16384
    hnsw_m: int = 32
    hnsw_ef_search: int = 64
    use_gpu: bool = True
    apply_to_key_vector: bool = False
    use_fused_sparse: bool = False


def retrieval_config_from_dict(cfg: dict) -> RetrievalConfig:
    """Reference index.py:372-387."""
    defaults = RetrievalConfig()
    return RetrievalConfig(**{f: cfg.get(f, getattr(defaults, f)) for f in defaults.__dataclass_fields__})


class RoutingRetriever(nn.Module):
    """Causal top-k retrieval in address space (reference index.py:101-221, exact methods).

    The reference casts the addresses to ``config.dtype`` and calls causal_topk; this
    build does the same for every method name, all on the HIP kernel.
    """

    def __init__(self, config: RetrievalConfig | None = None):
        super().__init__()
        self.config = config or RetrievalConfig()

    def ensure_capacity(self, seq_len: int) -> None:
        self.config.max_seq_len = max(self.config.max_seq_len, int(seq_len))

    def resolve_method(self, seq_len: int) -> RetrievalMethod:
        return self.config.method if self.config.method != "auto" else "fused_causal"

    def forward(self, query: torch.Tensor, key: torch.Tensor, top_k: int | None = None,
                method: RetrievalMethod | None = None) -> torch.Tensor:
        k = top_k or self.config.top_k
        if query.shape != key.shape:
            raise ValueError(
                f"Retrieval query/key shape mismatch: query={tuple(query.shape)}, "
                f"key={tuple(key.shape)}."
            )
        self.ensure_capacity(query.shape[1])
        m = method or self.resolve_method(query.shape[1])
        if m not in ("fused_causal", "brute_force", "faiss_flat", "faiss_hnsw"):
            raise ValueError(f"Unknown retrieval method: {m}")
        idx = causal_topk(query, key, k, method="fused_causal", dtype=self.config.dtype)
        return idx.long()
