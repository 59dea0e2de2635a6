"""Per-token learned address vectors (mirrors routing_attention/models/learned_address.py
of the reference: LearnedAddressModule, PerLayerAddressBook and the config helpers, same
parameters and state_dict keys)."""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels import address as address_kernel


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
        ``normalize`` (reference learned_address.py:39-46).

        On a ROCm device with no gradient to carry, both projections and the normalisation
        run as one HIP kernel (``wf_address_project_fwd``); otherwise the PyTorch ops."""
        kp = self.k_addr_proj
        needs_grad = torch.is_grad_enabled() and (
            hidden.requires_grad or any(p.requires_grad for p in self.parameters()))
        if not needs_grad and address_kernel.supported(hidden, self.q_addr_proj.weight,
                                                       kp.weight if kp is not None else None):
            return address_kernel.address_project(
                hidden, self.q_addr_proj.weight, self.q_addr_proj.bias,
                kp.weight if kp is not None else None, kp.bias if kp is not None else None,
                normalize=self.normalize)
        q = self.q_addr_proj(hidden)
        k = self.k_addr_proj(hidden) if self.k_addr_proj is not None else q
        if self.normalize:
            q = F.normalize(q, dim=-1)
            k = F.normalize(k, dim=-1)
        return q, k

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        q, _ = self.forward_query_key(hidden)
        return q

    def retrieval_scores(self, hidden: torch.Tensor) -> torch.Tensor:
        """Dense (B, T, T) address similarity (reference learned_address.py:53-56). The
        retrieval itself never builds this matrix; Recall@K can use
        ``routing_attention.evaluation.recall.compute_recall_from_addresses`` instead."""
        q, k = self.forward_query_key(hidden)
        return torch.matmul(q, k.transpose(-2, -1))


class PerLayerAddressBook(nn.Module):
    """One LearnedAddressModule per transformer layer (reference learned_address.py:59-90)."""

    def __init__(
        self,
        n_layers: int,
        d_model: int,
        address_dim: int = 32,
        similarity: Literal["symmetric", "asymmetric"] = "asymmetric",
        normalize: bool = True,
    ):
        super().__init__()
        self.n_layers = n_layers
        self.addresses = nn.ModuleList([
            LearnedAddressModule(d_model=d_model, address_dim=address_dim, similarity=similarity,
                                 normalize=normalize)
            for _ in range(n_layers)
        ])

    def get_address(self, layer_idx: int) -> LearnedAddressModule:
        return self.addresses[layer_idx]

    def get_router(self, layer_idx: int) -> LearnedAddressModule:
        return self.get_address(layer_idx)

    def retrieval_scores(self, hidden: torch.Tensor, layer_idx: int) -> torch.Tensor:
        return self.get_address(layer_idx).retrieval_scores(hidden)


def build_address_book_from_config(config: dict) -> PerLayerAddressBook:
    """Address book from the ``learned_address`` and ``model`` config sections (reference
    learned_address.py:93-103)."""
    la_cfg = config.get("learned_address", {})
    model_cfg = config["model"]
    return PerLayerAddressBook(
        n_layers=model_cfg["n_layers"],
        d_model=model_cfg["d_model"],
        address_dim=la_cfg.get("address_dim", la_cfg.get("routing_dim", 32)),
        similarity=la_cfg.get("similarity", "asymmetric"),
        normalize=la_cfg.get("normalize", True),
    )


def attach_address_book_to_model(model: nn.Module, address_book: PerLayerAddressBook) -> None:
    """Point every attention layer of a TransformerLM at its address module (reference
    learned_address.py:106-112)."""
    model.address_book = address_book
    for layer_idx, block in enumerate(model.blocks):
        if hasattr(block.attn, "set_address_module"):
            block.attn.set_address_module(address_book.get_address(layer_idx))
