from routing_attention.models.attention import LearnedAddressSparseAttention
from routing_attention.models.learned_address import LearnedAddressModule

__all__ = ["LearnedAddressSparseAttention", "LearnedAddressModule"]
