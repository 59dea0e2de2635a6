"""Routing projections whose vectors feed the causal top-K retrieval (mirrors
routing_attention/models/router.py of the reference: RouterMLP, PerLayerRouter,
MultiScaleRouter and build_router_from_config with the same parameters, state_dict keys
and outputs).

The routers themselves are small MLPs (torch Linear/GELU on the GPU). What changes on
MI355X is the retrieval behind them: ``retrieve_indices`` and every caller of
``forward_query_key`` select neighbours with the HIP causal top-K kernel, never through a
(B, T, T) score matrix.
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels.causal_topk import causal_topk


class RouterMLP(nn.Module):
    """Hidden states -> routing vectors (reference router.py:12-115).

    symmetric: one vector r_i, similarity r_i . r_j; asymmetric: separate query/key nets.
    With ``per_head_routing`` the output is (B, T, n_heads, routing_dim).
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
        hidden_dim = hidden_dim or max(routing_dim * 2, input_dim // 4)
        self.normalize = normalize
        self.use_affine_dot = use_affine_dot
        self.similarity = similarity
        self.n_heads = n_heads
        self.per_head_routing = per_head_routing
        self.routing_dim = routing_dim
        out_dim = routing_dim * n_heads if per_head_routing else routing_dim

        def mlp() -> nn.Sequential:
            return nn.Sequential(nn.Linear(input_dim, hidden_dim), nn.GELU(), nn.Dropout(dropout),
                                 nn.Linear(hidden_dim, out_dim))

        self.net = mlp()
        if similarity == "asymmetric":
            self.key_net = mlp()
        if use_affine_dot:
            self.dot_scale = nn.Parameter(torch.tensor(1.0))
            self.dot_bias = nn.Parameter(torch.tensor(0.0))

    def forward(self, x: torch.Tensor, as_query: bool = True) -> torch.Tensor:
        """(B, T, input_dim) -> (B, T, R), or (B, T, H, R) per head (reference :60-77)."""
        r = self.key_net(x) if (self.similarity == "asymmetric" and not as_query) else self.net(x)
        if self.per_head_routing:
            B, T, _ = r.shape
            r = r.view(B, T, self.n_heads, self.routing_dim)
        if self.normalize:
            r = F.normalize(r, dim=-1)
        return r

    def forward_query_key(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(query routing, key routing); the same tensor twice when symmetric (:79-86)."""
        q = self.forward(x, as_query=True)
        k = self.forward(x, as_query=False) if self.similarity == "asymmetric" else q
        return q, k

    def pairwise_scores(self, routing: torch.Tensor,
                        key_routing: torch.Tensor | None = None) -> torch.Tensor:
        """Dense pairwise scores for the routing losses (reference :88-103)."""
        key_routing = routing if key_routing is None else key_routing
        if routing.dim() == 4:
            # (B, T, H, R): per-head (B, H, T, S) scores, then the reference's .mean(dim=2),
            # which averages over the query axis T (reference :97-98), kept as is
            scores = torch.matmul(routing.permute(0, 2, 1, 3),
                                  key_routing.permute(0, 2, 3, 1).contiguous()).mean(dim=2)
        else:
            scores = torch.matmul(routing, key_routing.transpose(-2, -1))
        if self.use_affine_dot:
            scores = scores * self.dot_scale + self.dot_bias
        return scores

    def retrieval_scores(self, x: torch.Tensor) -> torch.Tensor:
        """Dense (B, T, T) similarity sim(query_i, key_j) (reference :105-115)."""
        q, k = self.forward_query_key(x)
        if q.dim() == 4:
            return torch.matmul(q.permute(0, 2, 1, 3),
                                k.permute(0, 2, 3, 1).contiguous()).sum(dim=1) / q.shape[2]
        return torch.matmul(q, k.transpose(-2, -1))


class PerLayerRouter(nn.Module):
    """One RouterMLP per transformer layer (reference router.py:118-156)."""

    def __init__(
        self,
        n_layers: int,
        input_dim: int,
        routing_dim: int = 32,
        hidden_dim: int | None = None,
        normalize: bool = True,
        use_affine_dot: bool = False,
        similarity: str = "symmetric",
        n_heads: int = 1,
        per_head_routing: bool = False,
    ):
        super().__init__()
        self.n_layers = n_layers
        self.routers = nn.ModuleList([
            RouterMLP(input_dim, routing_dim, hidden_dim, normalize, use_affine_dot=use_affine_dot,
                      similarity=similarity, n_heads=n_heads, per_head_routing=per_head_routing)
            for _ in range(n_layers)
        ])

    def forward(self, x: torch.Tensor, layer_idx: int, as_query: bool = True) -> torch.Tensor:
        return self.routers[layer_idx](x, as_query=as_query)

    def forward_query_key(self, x: torch.Tensor, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.routers[layer_idx].forward_query_key(x)

    def retrieval_scores(self, x: torch.Tensor, layer_idx: int) -> torch.Tensor:
        return self.routers[layer_idx].retrieval_scores(x)

    def get_router(self, layer_idx: int) -> RouterMLP:
        return self.routers[layer_idx]


def merge_candidate_sets(a: torch.Tensor, b: torch.Tensor, k: int) -> torch.Tensor:
    """Per row: the distinct values of a and b in ascending order, first k kept, short rows
    filled with the row's smallest value -- the loop of reference router.py:195-204
    (``cat(...).unique()[:k]``, tail = ``candidates[0]``), vectorised.

    a: (B, T, ka), b: (B, T, kb) integer tensors -> (B, T, k) int64.
    """
    c = torch.cat([a.long(), b.long()], dim=-1).sort(dim=-1).values
    first = torch.ones_like(c, dtype=torch.bool)
    first[..., 1:] = c[..., 1:] != c[..., :-1]
    # stable-sort the distinct entries to the front (their ascending order is kept)
    order = torch.argsort((~first).to(torch.int8), dim=-1, stable=True)
    uniq = torch.gather(c, -1, order)
    n_uniq = first.sum(dim=-1, keepdim=True)
    width = c.shape[-1]
    if width < k:
        uniq = torch.cat([uniq, uniq[..., :1].expand(*uniq.shape[:-1], k - width)], dim=-1)
    uniq = uniq[..., :k]
    slot = torch.arange(k, device=c.device).view(1, 1, k)
    return torch.where(slot < n_uniq, uniq, uniq[..., :1])


class MultiScaleRouter(nn.Module):
    """Local + global routers with merged candidate sets (reference router.py:159-207)."""

    def __init__(
        self,
        input_dim: int,
        routing_dim: int = 32,
        hidden_dim: int | None = None,
        local_window: int = 16,
        similarity: str = "symmetric",
        n_heads: int = 1,
        per_head_routing: bool = False,
    ):
        super().__init__()
        hidden_dim = hidden_dim or max(routing_dim * 2, input_dim // 4)
        self.local_window = local_window
        kw = dict(similarity=similarity, n_heads=n_heads, per_head_routing=per_head_routing)
        self.local_router = RouterMLP(input_dim, routing_dim, hidden_dim, normalize=True, **kw)
        self.global_router = RouterMLP(input_dim, routing_dim, hidden_dim, normalize=True, **kw)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch.cat([self.local_router(x), self.global_router(x)], dim=-1)

    @staticmethod
    def _topk_from_router(router: RouterMLP, x: torch.Tensor, k_eff: int) -> torch.Tensor:
        """Causal top-k of one router's similarity (reference :182-188) on the HIP kernel.
        Rows t < k_eff - 1 carry the kernel's pad indices where the reference's dense topk
        returns whichever -inf columns torch picks."""
        q, k = router.forward_query_key(x)
        if q.dim() == 4:
            raise ValueError("per-head routing vectors are (B,T,H,R); causal_topk takes (B,T,R)")
        return causal_topk(q, k, k_eff).long()

    def retrieve_indices(self, x: torch.Tensor, k: int, layer_idx: int = 0) -> torch.Tensor:
        """k/2 local + k - k/2 global candidates, merged (reference :190-204)."""
        del layer_idx
        k_half = max(1, k // 2)
        idx_local = self._topk_from_router(self.local_router, x, k_half)
        idx_global = self._topk_from_router(self.global_router, x, k - k_half)
        return merge_candidate_sets(idx_local, idx_global, k)

    def routing_for_loss(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return self.local_router(x), self.global_router(x)


def build_router_from_config(config: dict) -> nn.Module:
    """Single RouterMLP, PerLayerRouter or MultiScaleRouter from a config dict (reference
    router.py:210-253: same keys and defaults)."""
    router_cfg = config.get("router", {})
    model_cfg = config.get("model", {})
    mode = router_cfg.get("mode", "per_layer")
    input_dim = model_cfg["d_model"]
    routing_dim = router_cfg.get("routing_dim", 32)
    hidden_dim = router_cfg.get("hidden_dim")
    loss_type = router_cfg.get("loss_type", "infonce")
    normalize = loss_type not in ("mse",)
    use_affine_dot = loss_type == "mse"
    common = dict(similarity=router_cfg.get("similarity", "symmetric"),
                  n_heads=model_cfg.get("n_heads", 4),
                  per_head_routing=router_cfg.get("per_head_routing", False))
    if mode == "multi_scale":
        return MultiScaleRouter(input_dim=input_dim, routing_dim=routing_dim, hidden_dim=hidden_dim,
                                local_window=router_cfg.get("local_window", 16), **common)
    if mode == "per_layer":
        return PerLayerRouter(n_layers=model_cfg["n_layers"], input_dim=input_dim,
                              routing_dim=routing_dim, hidden_dim=hidden_dim, normalize=normalize,
                              use_affine_dot=use_affine_dot, **common)
    return RouterMLP(input_dim, routing_dim, hidden_dim, normalize=normalize,
                     use_affine_dot=use_affine_dot, **common)
