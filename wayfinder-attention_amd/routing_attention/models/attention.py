"""LearnedAddressSparseAttention on MI355X (mirrors the reference class in
routing_attention/models/attention.py:409-501: same constructor, forward signature,
submodules and state_dict keys).

With ``retrieval_config.use_fused_sparse`` the forward runs the fused HIP path
(wf_fused_topk_sparse_fwd): retrieval and readout in one library call, no autograd, as
the reference's @torch.no_grad fused_sparse_attention. The output is written directly in
(B, T, H, D) memory so the head merge before out_proj is a view, not a copy.
"""

from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels.fused_sparse import (
    fused_sparse_attention_bthd,
    sparse_meat_attention,
)
from routing_attention.models.learned_address import LearnedAddressModule
from routing_attention.retrieval.index import (
    RetrievalConfig,
    RoutingRetriever,
    retrieval_config_from_dict,
)


def _resolve_retrieval_cfg(retrieval_config: RetrievalConfig | dict | None,
                           top_k: int) -> RetrievalConfig:
    # reference attention.py:22-28
    if isinstance(retrieval_config, dict):
        return retrieval_config_from_dict(retrieval_config)
    return retrieval_config or RetrievalConfig(top_k=top_k)


def _use_fused_sparse_path(cfg: RetrievalConfig | None) -> bool:
    # reference attention.py:31-32
    return bool(cfg and cfg.use_fused_sparse)


def _sparse_readout_autograd(q, k, v, idx, scale, dropout: nn.Dropout) -> torch.Tensor:
    """Differentiable readout for the training path (reference attention.py:50-55). The
    HIP readout has no backward yet, so gradients flow through this gather formulation."""
    B, H = k.shape[0], k.shape[1]
    bi = torch.arange(B, device=k.device).view(B, 1, 1, 1)
    hi = torch.arange(H, device=k.device).view(1, H, 1, 1)
    ii = idx.long().unsqueeze(1)
    k_sel, v_sel = k[bi, hi, ii, :], v[bi, hi, ii, :]
    scores = (q.unsqueeze(3) * k_sel).sum(-1) * scale
    attn = dropout(F.softmax(scores, dim=-1))
    return (attn.unsqueeze(-1) * v_sel).sum(dim=3)


class LearnedAddressSparseAttention(nn.Module):
    """Sparse attention: learned addresses pick K candidates per token; Q/K/V attention
    runs on that subset (reference attention.py:409-501)."""

    def __init__(
        self,
        d_model: int,
        n_heads: int,
        top_k: int = 32,
        address_dim: int = 32,
        similarity: Literal["symmetric", "asymmetric"] = "asymmetric",
        dropout: float = 0.1,
        address_module: LearnedAddressModule | None = None,
        retrieval_config: RetrievalConfig | dict | None = None,
    ):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.scale = self.head_dim ** -0.5
        self.top_k = top_k
        self._retrieval_cfg = _resolve_retrieval_cfg(retrieval_config, top_k)
        self.retriever = RoutingRetriever(self._retrieval_cfg)
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)
        self.dropout = nn.Dropout(dropout)
        self.address = address_module or LearnedAddressModule(
            d_model=d_model, address_dim=address_dim, similarity=similarity
        )

    def set_address_module(self, address_module: LearnedAddressModule) -> None:
        self.address = address_module

    def _retrieve_candidates(self, x: torch.Tensor) -> torch.Tensor:
        q_addr, k_addr = self.address.forward_query_key(x)
        return self.retriever(q_addr, k_addr, top_k=self.top_k)

    def forward(
        self,
        x: torch.Tensor,
        attn_mask: Optional[torch.Tensor] = None,
        return_attention: bool = False,
        **kwargs,
    ) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
        """x (B, T, d_model) -> (B, T, d_model). attn_mask is ignored (causality comes
        from the retrieval), as in the reference."""
        del attn_mask, kwargs
        B, T, D = x.shape
        H, hd = self.n_heads, self.head_dim
        q = self.q_proj(x).view(B, T, H, hd).transpose(1, 2)
        k = self.k_proj(x).view(B, T, H, hd).transpose(1, 2)
        v = self.v_proj(x).view(B, T, H, hd).transpose(1, 2)

        if _use_fused_sparse_path(self._retrieval_cfg):
            q_addr, k_addr = self.address.forward_query_key(x)
            meat_bthd, candidate_idx = fused_sparse_attention_bthd(
                q_addr, k_addr, q, k, v, self.top_k, self.scale
            )
            out = meat_bthd.view(B, T, D)
        else:
            candidate_idx = self._retrieve_candidates(x)
            needs_grad = torch.is_grad_enabled() and (
                q.requires_grad or k.requires_grad or v.requires_grad
            )
            if needs_grad or (self.training and self.dropout.p > 0):
                meat = _sparse_readout_autograd(q, k, v, candidate_idx, self.scale, self.dropout)
            else:
                meat = sparse_meat_attention(q, k, v, candidate_idx, self.scale)
            out = meat.transpose(1, 2).contiguous().view(B, T, D)

        out = self.out_proj(out)
        if return_attention:
            k_eff = candidate_idx.shape[-1]
            attn_dense = torch.zeros(B, T, T, device=x.device)
            if k_eff:
                attn_dense.scatter_(2, candidate_idx.long(), 1.0 / k_eff)
            return out, attn_dense
        return out
