"""MI355X kernels for causal top-K retrieval and fused sparse attention.

Same public names as the reference's routing_attention/kernels/__init__.py:3-23.
"""

from routing_attention.kernels.fused_sparse import (
    SparseMeatConfig,
    fused_sparse_attention,
    fused_sparse_attention_available,
    sparse_meat_attention,
)
from routing_attention.kernels.causal_topk import (
    causal_topk,
    causal_topk_available,
    causal_topk_reference,
)

__all__ = [
    "causal_topk",
    "causal_topk_available",
    "causal_topk_reference",
    "SparseMeatConfig",
    "sparse_meat_attention",
    "fused_sparse_attention",
    "fused_sparse_attention_available",
]
