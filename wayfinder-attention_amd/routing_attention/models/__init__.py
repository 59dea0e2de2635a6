"""Model-side mirror of the reference's routing_attention/models/__init__.py for the
modules on the top-K sparse-attention path (the dense comparator included)."""

from routing_attention.models.attention import (
    DenseSDPAAttention,
    KeyVectorSparseAttention,
    LearnedAddressSparseAttention,
    RoutingSparseAttention,
)
from routing_attention.models.learned_address import (
    LearnedAddressModule,
    PerLayerAddressBook,
    build_address_book_from_config,
)
from routing_attention.models.router import RouterMLP
from routing_attention.models.transformer import TransformerBlock, TransformerLM

__all__ = [
    "DenseSDPAAttention",
    "KeyVectorSparseAttention",
    "LearnedAddressModule",
    "LearnedAddressSparseAttention",
    "PerLayerAddressBook",
    "RouterMLP",
    "RoutingSparseAttention",
    "TransformerBlock",
    "TransformerLM",
    "build_address_book_from_config",
]
