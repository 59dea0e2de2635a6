"""Retrieval evaluation on the streaming top-K (mirrors routing_attention/evaluation/recall.py
of the reference for Recall@K, ``compute_recall_at_k``)."""

from routing_attention.evaluation.recall import (
    compute_recall_at_k,
    compute_recall_from_addresses,
    compute_recall_from_vectors,
)

__all__ = [
    "compute_recall_at_k",
    "compute_recall_from_addresses",
    "compute_recall_from_vectors",
]
