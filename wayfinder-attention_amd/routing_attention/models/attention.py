"""Sparse attention modules on MI355X (mirror routing_attention/models/attention.py of the
reference for the three classes on the top-K path -- LearnedAddressSparseAttention
(:409-501), KeyVectorSparseAttention (:296-406) and RoutingSparseAttention (:504-617) --
plus DenseSDPAAttention (:130-173), the dense comparator. Same constructors, forward
signatures, submodules and state_dict keys).

With ``retrieval_config.use_fused_sparse`` each forward runs the fused HIP path
(wf_fused_topk_sparse_fwd): retrieval and readout in one library call, no autograd, as the
reference's @torch.no_grad fused_sparse_attention. Its output is written directly in
(B, T, H, D) memory, so the head merge before out_proj is a view, not a copy. The other
branch retrieves with the HIP causal top-K and reads out with the HIP readout, forward and
backward, dropout in training included (inside the readout kernels).
"""

from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels.causal_topk import causal_topk
from routing_attention.kernels.fused_sparse import (
    fused_sparse_attention_bthd,
    sparse_meat_attention,
)
from routing_attention.kernels.sparse_autograd import sparse_readout
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


def _sparse_meat_forward(q, k, v, candidate_idx, scale: float, dropout: nn.Dropout,
                         cfg: RetrievalConfig | None) -> torch.Tensor:
    """Attention of each query over its K candidates, (B, H, T, D) (reference
    attention.py:35-55).

    * dropout active (training with p > 0): ``sparse_readout`` with dropout on the
      attention weights after the softmax, as the reference's non-fused branch, in the
      HIP forward and backward (the keep mask is a hash of a seed drawn from torch's
      generator, recomputed by the backward; nothing of size (B, H, T, K, D) is formed);
    * a gradient is needed: ``sparse_readout``, the HIP forward and backward (dq by a
      row pass, dk/dv over the transposed index lists, deterministic);
    * otherwise: the no-grad HIP readout ``sparse_meat_attention``.
    """
    del cfg
    if dropout.training and dropout.p > 0:
        return sparse_readout(q, k, v, candidate_idx, scale, dropout_p=dropout.p)
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if needs_grad:
        return sparse_readout(q, k, v, candidate_idx, scale)
    return sparse_meat_attention(q, k, v, candidate_idx, scale)


def _fused_merged(q_search, k_search, q, k, v, top_k: int, scale: float):
    """Fused retrieval + readout; returns ((B, T, H*D) head-merged output view, indices)."""
    B, _, T, _ = q.shape
    meat_bthd, idx = fused_sparse_attention_bthd(q_search, k_search, q, k, v, top_k, scale)
    return meat_bthd.view(B, T, -1), idx


def _merge_heads(meat: torch.Tensor) -> torch.Tensor:
    B, H, T, D = meat.shape
    return meat.transpose(1, 2).contiguous().view(B, T, H * D)


def _dense_attention_map(candidate_idx: torch.Tensor, T: int) -> torch.Tensor:
    """(B, T, T) map with 1/k_eff at every selected (query, key) pair -- the triple loop of
    reference attention.py:396-405, as one scatter."""
    B = candidate_idx.shape[0]
    k_eff = candidate_idx.shape[-1]
    attn_dense = torch.zeros(B, T, T, device=candidate_idx.device)
    if k_eff:
        attn_dense.scatter_(2, candidate_idx.long(), 1.0 / k_eff)
    return attn_dense


def _qkv(module: nn.Module, x: torch.Tensor):
    """(B, T, d_model) -> q, k, v as (B, H, T, hd) views of (B, T, H, hd) memory."""
    B, T, _ = x.shape
    H, hd = module.n_heads, module.head_dim
    q = module.q_proj(x).view(B, T, H, hd).transpose(1, 2)
    k = module.k_proj(x).view(B, T, H, hd).transpose(1, 2)
    v = module.v_proj(x).view(B, T, H, hd).transpose(1, 2)
    return q, k, v


class DenseSDPAAttention(nn.Module):
    """Dense causal attention through F.scaled_dot_product_attention (reference
    attention.py:130-173; same projections as the sparse modules). The comparator the
    sparse path is measured against."""

    def __init__(self, d_model: int, n_heads: int, dropout: float = 0.1):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_attention: bool = False, **kwargs) -> torch.Tensor:
        if return_attention:
            raise NotImplementedError("dense attention weights are outside this build's scope")
        del kwargs
        B, T, D = x.shape
        q, k, v = _qkv(self, x)
        sdpa_mask = None
        if attn_mask is not None:   # reference :156-160: padding mask & causal
            causal = torch.tril(torch.ones(T, T, device=x.device, dtype=torch.bool))
            sdpa_mask = attn_mask.bool().view(B, 1, 1, T) & causal.view(1, 1, T, T)
        out = F.scaled_dot_product_attention(
            q, k, v, attn_mask=sdpa_mask, dropout_p=self.dropout.p if self.training else 0.0,
            is_causal=sdpa_mask is None, scale=self.scale)
        return self.out_proj(_merge_heads(out))


class KeyVectorSparseAttention(nn.Module):
    """kNN on key vectors: candidates by the head-mean Q/K geometry (reference
    attention.py:296-406).

    Retrieval policy: ``apply_to_key_vector=False`` (default) takes the inline exact top-K;
    ``True`` goes through RoutingRetriever (its dtype cast first). Both run the HIP causal
    top-K on fp32 scores of the search vectors; the reference's inline path ranks bf16/fp16
    matmul scores, so near-ties within that rounding may resolve differently.
    """

    def __init__(
        self,
        d_model: int,
        n_heads: int,
        top_k: int = 32,
        dropout: float = 0.1,
        retrieval_config: RetrievalConfig | dict | None = None,
    ):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.scale = self.head_dim ** -0.5
        self.top_k = top_k
        self._retrieval_cfg = _resolve_retrieval_cfg(retrieval_config, top_k)
        self.use_fast_retrieval = self._retrieval_cfg.apply_to_key_vector
        self.retriever = (
            RoutingRetriever(self._retrieval_cfg)
            if self.use_fast_retrieval or self._retrieval_cfg.use_fused_sparse
            else None
        )
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)
        self.dropout = nn.Dropout(dropout)

    def _search_vectors(self, k: torch.Tensor, q: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Head means used only for index selection (reference :339-341). The parameter
        order and every call site follow the reference, so the "query" search vector is
        the head-mean of the keys and the "key" search vector the head-mean of the queries,
        exactly as there."""
        return q.mean(dim=1), k.mean(dim=1)

    def _retrieve_by_keys_inline(self, k: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
        """Exact causal top-K of the search vectors (reference :343-352)."""
        q_mean, k_mean = self._search_vectors(q, k)
        return causal_topk(q_mean, k_mean, self.top_k).long()

    def _retrieve_by_keys(self, k: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
        # reference :354-359
        if not self.use_fast_retrieval:
            return self._retrieve_by_keys_inline(k, q)
        q_mean, k_mean = self._search_vectors(q, k)
        return self.retriever(q_mean, k_mean, top_k=self.top_k)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_attention: bool = False, **kwargs):
        del attn_mask, kwargs
        B, T, D = x.shape
        q, k, v = _qkv(self, x)
        if _use_fused_sparse_path(self._retrieval_cfg):
            q_mean, k_mean = self._search_vectors(q, k)
            out, candidate_idx = _fused_merged(q_mean, k_mean, q, k, v, self.top_k, self.scale)
        else:
            candidate_idx = self._retrieve_by_keys(k, q)
            meat = _sparse_meat_forward(q, k, v, candidate_idx, self.scale, self.dropout,
                                        self._retrieval_cfg)
            out = _merge_heads(meat)
        out = self.out_proj(out)
        if return_attention:
            return out, _dense_attention_map(candidate_idx, T)
        return out


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
        q, k, v = _qkv(self, x)
        if _use_fused_sparse_path(self._retrieval_cfg):
            q_addr, k_addr = self.address.forward_query_key(x)
            out, candidate_idx = _fused_merged(q_addr, k_addr, q, k, v, self.top_k, self.scale)
        else:
            candidate_idx = self._retrieve_candidates(x)
            meat = _sparse_meat_forward(q, k, v, candidate_idx, self.scale, self.dropout,
                                        self._retrieval_cfg)
            out = _merge_heads(meat)
        out = self.out_proj(out)
        if return_attention:
            return out, _dense_attention_map(candidate_idx, T)
        return out


class RoutingSparseAttention(nn.Module):
    """Sparse attention with router vectors for retrieval (reference attention.py:504-617).
    The router is a RouterMLP, a per-layer container (anything with ``get_router``, picked
    by layer_idx) or a candidate generator of its own (anything with ``retrieve_indices``,
    the reference's multi-scale router)."""

    def __init__(
        self,
        d_model: int,
        n_heads: int,
        router: nn.Module,
        top_k: int = 32,
        dropout: float = 0.1,
        layer_idx: int = 0,
        retrieval_mode: Literal["routing", "key_vector"] = "routing",
        retrieval_config: RetrievalConfig | dict | None = None,
    ):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.scale = self.head_dim ** -0.5
        self.top_k = top_k
        self.router = router
        self.layer_idx = layer_idx
        self.retrieval_mode = retrieval_mode
        self._retrieval_cfg = _resolve_retrieval_cfg(retrieval_config, top_k)
        self.retriever = RoutingRetriever(self._retrieval_cfg)
        self._last_retrieval_ms: float = 0.0
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)
        self.dropout = nn.Dropout(dropout)
        if retrieval_mode == "key_vector":
            self._key_baseline = KeyVectorSparseAttention(
                d_model, n_heads, top_k, dropout, retrieval_config=retrieval_config
            )

    def _get_query_key_routing(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(query, key) routing vectors of this layer (reference :548-555)."""
        router = self.router.get_router(self.layer_idx) if hasattr(self.router, "get_router") else self.router
        if hasattr(router, "forward_query_key"):
            return router.forward_query_key(x)
        r = router(x)
        return r, r

    def _retrieve_candidates(self, x: torch.Tensor) -> torch.Tensor:
        """(B, T, top_k) neighbours: the router's own candidate generator if it has one,
        else the causal top-K of its vectors (reference :557-566)."""
        if hasattr(self.router, "retrieve_indices"):
            return self.router.retrieve_indices(x, self.top_k, self.layer_idx)
        q, k = self._get_query_key_routing(x)
        return self.retriever(q, k, top_k=self.top_k)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_attention: bool = False,
                precomputed_routing: Optional[torch.Tensor] = None, **kwargs):
        del precomputed_routing, kwargs
        if self.retrieval_mode == "key_vector":
            return self._key_baseline(x, attn_mask=attn_mask, return_attention=return_attention)
        B, T, D = x.shape
        q, k, v = _qkv(self, x)
        if _use_fused_sparse_path(self._retrieval_cfg):
            q_r, k_r = self._get_query_key_routing(x)
            out, candidate_idx = _fused_merged(q_r, k_r, q, k, v, self.top_k, self.scale)
        else:
            candidate_idx = self._retrieve_candidates(x)
            meat = _sparse_meat_forward(q, k, v, candidate_idx, self.scale, self.dropout,
                                        self._retrieval_cfg)
            out = _merge_heads(meat)
        out = self.out_proj(out)
        if return_attention:
            return out, _dense_attention_map(candidate_idx, T)
        return out
