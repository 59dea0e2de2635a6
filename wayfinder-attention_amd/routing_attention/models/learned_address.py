"""Per-token learned address vectors (the reference's routing_attention/models/
learned_address.py: LearnedAddressModule :12-56 and the per-layer book :59-103, with the
same constructor arguments, parameter names and state_dict keys).

Addresses are the only input of the retrieval: q_addr = normalize(W_q x + b_q) and
k_addr = normalize(W_k x + b_k) (one projection when symmetric). Without a gradient to
carry, both projections and the normalisation run as one HIP kernel
(wf_address_project_fwd). Phase-B scoring of the addresses has two forms: the reference's
dense (B, T, T) ``retrieval_scores`` and ``retrieval_topk``, the causal top-K rows of the
same scores from the HIP streaming top-K, which never forms the (B, T, T) matrix.
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels import address as address_kernel
from routing_attention.kernels.causal_topk import causal_topk_with_scores


class LearnedAddressModule(nn.Module):
    """Hidden states (B, T, d_model) -> (query, key) addresses (B, T, address_dim) used only
    to choose neighbours."""

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

    def _needs_graph(self, hidden: torch.Tensor) -> bool:
        return torch.is_grad_enabled() and (
            hidden.requires_grad or any(p.requires_grad for p in self.parameters()))

    def forward_query_key(self, hidden: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Both addresses, L2-normalised when ``normalize`` (reference
        learned_address.py:39-46). On a ROCm device with no gradient to carry: one HIP
        kernel; otherwise the PyTorch ops, so autograd sees the graph."""
        kp = self.k_addr_proj
        kw = kp.weight if kp is not None else None
        if not self._needs_graph(hidden) and address_kernel.supported(hidden, self.q_addr_proj.weight, kw):
            return address_kernel.address_project(
                hidden, self.q_addr_proj.weight, self.q_addr_proj.bias, kw,
                kp.bias if kp is not None else None, normalize=self.normalize)
        heads = [self.q_addr_proj(hidden)]
        if kp is not None:
            heads.append(kp(hidden))
        if self.normalize:
            heads = [F.normalize(a, dim=-1) for a in heads]
        return heads[0], heads[-1]

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.forward_query_key(hidden)[0]

    def retrieval_scores(self, hidden: torch.Tensor) -> torch.Tensor:
        """Dense (B, T, T) address similarity q_addr_i . k_addr_j (reference
        learned_address.py:53-56). Prefer retrieval_topk, which never forms it."""
        q, k = self.forward_query_key(hidden)
        return torch.matmul(q, k.transpose(-2, -1).contiguous())

    @torch.no_grad()
    def retrieval_topk(self, hidden: torch.Tensor, top_k: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The causal top-K of each row of retrieval_scores: int32 indices (B, T, k_eff) in
        canonical order (score descending, ties to the lower index, pads last) and their fp32
        scores (-inf in pad slots), from the HIP streaming top-K."""
        q, k = self.forward_query_key(hidden)
        return causal_topk_with_scores(q, k, top_k)


class PerLayerAddressBook(nn.Module):
    """One LearnedAddressModule per transformer layer (reference learned_address.py:59-90);
    state_dict keys ``addresses.<layer>.q_addr_proj.weight`` etc."""

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
        self.addresses = nn.ModuleList(
            LearnedAddressModule(d_model, address_dim, similarity, normalize) for _ in range(n_layers))

    def get_address(self, layer_idx: int) -> LearnedAddressModule:
        return self.addresses[layer_idx]

    # the routers' accessor name, so code written for per-layer routers takes a book too
    get_router = get_address

    def retrieval_scores(self, hidden: torch.Tensor, layer_idx: int) -> torch.Tensor:
        return self.addresses[layer_idx].retrieval_scores(hidden)

    def retrieval_topk(self, hidden: torch.Tensor, layer_idx: int,
                       top_k: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.addresses[layer_idx].retrieval_topk(hidden, top_k)


def build_address_book_from_config(config: dict) -> PerLayerAddressBook:
    """PerLayerAddressBook from a config dict: ``model.n_layers`` / ``model.d_model`` and the
    ``learned_address`` section's address_dim (alias routing_dim, default 32), similarity
    (default asymmetric) and normalize (default True) -- the reference's keys and defaults
    (learned_address.py:93-103)."""
    section = config.get("learned_address") or {}
    dim = section["address_dim"] if "address_dim" in section else section.get("routing_dim", 32)
    return PerLayerAddressBook(
        config["model"]["n_layers"], config["model"]["d_model"], address_dim=dim,
        similarity=section.get("similarity", "asymmetric"), normalize=section.get("normalize", True))
