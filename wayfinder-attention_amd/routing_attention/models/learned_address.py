"""Per-token learned address vectors (mirrors routing_attention/models/learned_address.py
of the reference: LearnedAddressModule, same parameters and state_dict keys)."""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F


class LearnedAddressModule(nn.Module):
    """Maps hidden states to (query, key) addresses of dim ``address_dim`` used only for
    retrieval (reference learned_address.py:12-56)."""

    def __init__(
        self,
        d_model: int,
        address_dim: int = 32,
        similarity: Literal["symmetric", "asymmetric"] = "asymmetric",
        normalize: bool = True,
    ):
        super().__init__()
        self.d_model = d_model
        self.address_dim = address_dim
        self.similarity = similarity
        self.normalize = normalize
        self.q_addr_proj = nn.Linear(d_model, address_dim)
        self.k_addr_proj = nn.Linear(d_model, address_dim) if similarity == "asymmetric" else None

    def forward_query_key(self, hidden: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(B, T, d_model) -> two (B, T, address_dim) addresses, L2-normalised when
        ``normalize`` (reference learned_address.py:39-46)."""
        q = self.q_addr_proj(hidden)
        k = self.k_addr_proj(hidden) if self.k_addr_proj is not None else q
        if self.normalize:
            q = F.normalize(q, dim=-1)
            k = F.normalize(k, dim=-1)
        return q, k

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        q, _ = self.forward_query_key(hidden)
        return q
