"""Retrieval evaluation on the streaming top-K (mirrors routing_attention/evaluation/recall.py
of the reference for the Recall@K functions)."""

from routing_attention.evaluation.recall import (
    compute_key_vector_recall_from_hidden,
    compute_recall_at_k,
    compute_recall_by_distance,
    compute_recall_by_distance_from_router,
    compute_recall_from_router,
    compute_recall_from_vectors,
)

__all__ = [
    "compute_key_vector_recall_from_hidden",
    "compute_recall_at_k",
    "compute_recall_by_distance",
    "compute_recall_by_distance_from_router",
    "compute_recall_from_router",
    "compute_recall_from_vectors",
]
