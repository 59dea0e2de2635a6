"""Routing vectors for RoutingSparseAttention (the reference's RouterMLP,
routing_attention/models/router.py:12-115: same constructor, submodule names and
state_dict keys, so its checkpoints load unchanged).

A router maps hidden states to unit-norm routing vectors; the causal top-K over their dot
products picks each token's neighbours. Only the single-network router is part of this
build; the per-layer and multi-scale containers of the reference are outside the hot path
(RoutingSparseAttention still accepts any object with ``get_router(layer_idx)`` or
``retrieve_indices(...)``).
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels.causal_topk import causal_topk_with_scores


def _routing_mlp(d_in: int, d_hidden: int, d_out: int, p: float) -> nn.Sequential:
    # Linear -> GELU -> Dropout -> Linear; the positions (0 and 3) are part of the
    # state_dict key names of the reference ("net.0.weight", "net.3.weight")
    return nn.Sequential(nn.Linear(d_in, d_hidden), nn.GELU(), nn.Dropout(p), nn.Linear(d_hidden, d_out))


class RouterMLP(nn.Module):
    """Hidden states -> routing vectors.

    symmetric: one network, similarity r_i . r_j; asymmetric: a second network for keys.
    per_head_routing: n_heads vectors of routing_dim per token, (B, T, H, R); their
    similarity is the head mean of the per-head dot products.
    """

    def __init__(
        self,
        input_dim: int,
        routing_dim: int = 32,
        hidden_dim: int | None = None,
        normalize: bool = True,
        dropout: float = 0.0,
        use_affine_dot: bool = False,
        similarity: Literal["symmetric", "asymmetric"] = "symmetric",
        n_heads: int = 1,
        per_head_routing: bool = False,
    ):
        super().__init__()
        width = hidden_dim if hidden_dim else max(2 * routing_dim, input_dim // 4)
        n_out = routing_dim * (n_heads if per_head_routing else 1)
        self.routing_dim = routing_dim
        self.n_heads = n_heads
        self.per_head_routing = per_head_routing
        self.normalize = normalize
        self.similarity = similarity
        self.use_affine_dot = use_affine_dot
        self.net = _routing_mlp(input_dim, width, n_out, dropout)
        if similarity == "asymmetric":
            self.key_net = _routing_mlp(input_dim, width, n_out, dropout)
        if use_affine_dot:
            self.dot_scale = nn.Parameter(torch.ones(()))
            self.dot_bias = nn.Parameter(torch.zeros(()))

    def _vectors(self, x: torch.Tensor, net: nn.Module) -> torch.Tensor:
        r = net(x)
        if self.per_head_routing:
            r = r.unflatten(-1, (self.n_heads, self.routing_dim))
        return F.normalize(r, dim=-1) if self.normalize else r

    def forward(self, x: torch.Tensor, as_query: bool = True) -> torch.Tensor:
        """(B, T, input_dim) -> (B, T, R), or (B, T, H, R) per head. Keys come from key_net
        when the router is asymmetric and ``as_query`` is False."""
        use_key_net = not as_query and self.similarity == "asymmetric"
        return self._vectors(x, self.key_net if use_key_net else self.net)

    def forward_query_key(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(query vectors, key vectors); one tensor twice when symmetric."""
        q = self._vectors(x, self.net)
        if self.similarity != "asymmetric":
            return q, q
        return q, self._vectors(x, self.key_net)

    def pairwise_scores(self, routing: torch.Tensor,
                        key_routing: torch.Tensor | None = None) -> torch.Tensor:
        """Dense scores for the routing losses (reference router.py:88-103). Per-head input
        gives (B, H, T, S) dot products averaged over the query axis, as the reference's
        ``.mean(dim=2)`` does; otherwise (B, T, S)."""
        keys = routing if key_routing is None else key_routing
        if routing.dim() == 4:
            s = torch.matmul(routing.transpose(1, 2), keys.permute(0, 2, 3, 1).contiguous()).mean(dim=2)
        else:
            s = torch.matmul(routing, keys.transpose(-2, -1))
        return s * self.dot_scale + self.dot_bias if self.use_affine_dot else s

    def retrieval_scores(self, x: torch.Tensor) -> torch.Tensor:
        """Dense (B, T, T) similarity of query i and key j (head mean for per-head vectors)
        (reference router.py:105-115). The retrieval never builds it; see retrieval_topk."""
        q, k = self.forward_query_key(x)
        h = q.shape[2] if q.dim() == 4 else 1
        return torch.matmul(q.flatten(2), k.flatten(2).transpose(-2, -1)) / h

    @torch.no_grad()
    def retrieval_topk(self, x: torch.Tensor, top_k: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The causal top-K rows of retrieval_scores without forming them: int32 indices
        (B, T, k_eff) in canonical order and their fp32 scores (-inf in pad slots), from the
        HIP streaming top-K. Per-head vectors are ranked by their concatenated dot product,
        which orders keys as the head mean does; the scores are divided by H to match it."""
        q, k = self.forward_query_key(x)
        h = q.shape[2] if q.dim() == 4 else 1
        idx, sc = causal_topk_with_scores(q.flatten(2), k.flatten(2), top_k)
        return idx, sc / h if h > 1 else sc
