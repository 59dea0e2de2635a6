"""Phase-B address-training loss on the retrieval path (mirrors the reference's
routing_attention/losses: batched_infonce_loss)."""

from routing_attention.losses.contrastive import batched_infonce_loss

__all__ = ["batched_infonce_loss"]
