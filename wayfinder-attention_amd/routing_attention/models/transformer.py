"""Decoder-only language model around the sparse attention modules (the reference's
routing_attention/models/transformer.py: TransformerBlock :26-73 and TransformerLM
:76-401). Kept from the reference, as interface: the constructor arguments, the submodule
names and hence the state_dict keys (token_emb, pos_emb, blocks.<i>.{ln1, attn, ln2, ff.0,
ff.3}, ln_f, lm_head tied to token_emb, digit_head), and the value of the masked
next-token loss.

Attention types here: ``learned_address``, ``key_vector`` and ``routing`` (the top-K sparse
modules: HIP retrieval and readout) and ``dense`` / ``dense_flash`` (causal SDPA, the
comparator). ``linear`` and ``local`` attention, the pointer / pool output heads and the
per-layer / multi-scale router configurations are outside this build and raise.
"""

from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.kernels import layernorm as _ln_kernel
from routing_attention.models.attention import (
    DenseSDPAAttention,
    KeyVectorSparseAttention,
    LearnedAddressSparseAttention,
    RoutingSparseAttention,
)
from routing_attention.models.learned_address import build_address_book_from_config
from routing_attention.models.router import RouterMLP


class TransformerBlock(nn.Module):
    """Pre-norm residual block: x + attn(ln1 x), then + ff(ln2 .) with a 4-module MLP
    (Linear, GELU, Dropout, Linear) followed by dropout."""

    def __init__(self, d_model: int, n_heads: int, d_ff: int, dropout: float,
                 attention_module: nn.Module, layer_idx: int = 0):
        super().__init__()
        del n_heads   # carried by the attention module
        self.layer_idx = layer_idx
        self.ln1 = nn.LayerNorm(d_model)
        self.attn = attention_module
        self.ln2 = nn.LayerNorm(d_model)
        self.ff = nn.Sequential(nn.Linear(d_model, d_ff), nn.GELU(), nn.Dropout(dropout),
                                nn.Linear(d_ff, d_model), nn.Dropout(dropout))

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_attention: bool = False, return_per_head: bool = False, **attn_kwargs):
        """Returns x, or (x, attention weights) with ``return_attention``."""
        if return_attention:
            attn_kwargs.update(return_attention=True, return_per_head=return_per_head)
        a = self.attn(self.ln1(x), attn_mask=attn_mask, **attn_kwargs)
        a, weights = a if return_attention else (a, None)
        x = x + a
        x = x + self.ff(self.ln2(x))
        return (x, weights) if return_attention else x


def _router_from_config(d_model: int, config: dict) -> RouterMLP:
    """The router a config asks for. Only its single-router mode is part of this build
    (the reference's default, per-layer, and its multi-scale mode are not)."""
    section = config.get("router") or {}
    mode = section.get("mode", "per_layer")
    if mode != "single":
        raise NotImplementedError(f"router mode {mode!r} is not part of this build; "
                                  "pass router=RouterMLP(...) instead")
    return RouterMLP(d_model, section.get("routing_dim", 32), section.get("hidden_dim"),
                     similarity=section.get("similarity", "symmetric"))


class TransformerLM(nn.Module):
    """Decoder-only transformer language model (token + learned position embeddings,
    pre-norm blocks, final LayerNorm, LM head tied to the token embedding)."""

    _SPARSE = ("learned_address", "key_vector", "routing")

    def __init__(
        self,
        vocab_size: int,
        d_model: int = 256,
        n_layers: int = 6,
        n_heads: int = 4,
        d_ff: int = 1024,
        max_seq_len: int = 512,
        dropout: float = 0.1,
        attention_type: Literal[
            "dense", "dense_flash", "linear", "local", "routing", "key_vector", "learned_address"
        ] = "dense",
        router: Optional[nn.Module] = None,
        routing_top_k: int = 32,
        local_window: int = 64,
        pad_token_id: int = 0,
        num_digit_classes: int = 0,
        output_head: Literal["lm_token", "pointer_index", "pointer_mlp", "pool_mlp_token"] = "lm_token",
        pointer_target_mode: Literal["value_slots", "full_sequence"] = "full_sequence",
        pointer_mlp_hidden: int = 2100,
        num_pointer_slots: int = 50,
        pool_mlp_positions: int = 16,
        config: Optional[dict] = None,
        retrieval_config: Optional[dict] = None,
    ):
        super().__init__()
        del local_window, pointer_mlp_hidden, num_pointer_slots, pool_mlp_positions
        if output_head != "lm_token":
            raise NotImplementedError(f"output_head={output_head!r} is not part of this build")
        if attention_type in ("linear", "local"):
            raise NotImplementedError(f"attention_type={attention_type!r} is not part of this build")
        if attention_type not in self._SPARSE + ("dense", "dense_flash"):
            raise ValueError(f"Unknown attention_type: {attention_type}")
        self.attention_type = attention_type
        self.d_model, self.n_layers, self.n_heads = d_model, n_layers, n_heads
        self.max_seq_len = max_seq_len
        self.pad_token_id = pad_token_id
        self.routing_top_k = routing_top_k
        self.output_head = output_head
        self.pointer_target_mode = pointer_target_mode
        self.retrieval_config = retrieval_config if retrieval_config is not None else (config or {}).get("retrieval")
        if attention_type == "routing" and router is None and config is not None:
            router = _router_from_config(d_model, config)
        self.router = router
        # without a router, the routing layers share one RouterMLP that only the blocks hold
        # (the model's own `router` stays None, as in the reference)
        shared = router
        if attention_type == "routing" and shared is None:
            shared = RouterMLP(d_model, routing_dim=32)
        self.address_book = (build_address_book_from_config(config)
                             if attention_type == "learned_address" and config is not None else None)

        self.token_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Embedding(max_seq_len, d_model)
        self.dropout = nn.Dropout(dropout)
        self.blocks = nn.ModuleList(
            TransformerBlock(d_model, n_heads, d_ff, dropout,
                             self._attention(i, d_model, n_heads, dropout, config, shared), layer_idx=i)
            for i in range(n_layers))
        self.ln_f = nn.LayerNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.token_emb.weight
        self.num_digit_classes = num_digit_classes
        self.digit_head = nn.Linear(d_model, num_digit_classes) if num_digit_classes > 0 else None

    def _attention(self, layer: int, d_model: int, n_heads: int, dropout: float,
                   config: Optional[dict], router: Optional[nn.Module]) -> nn.Module:
        kind, k, rc = self.attention_type, self.routing_top_k, self.retrieval_config
        if kind in ("dense", "dense_flash"):
            return DenseSDPAAttention(d_model, n_heads, dropout)
        if kind == "key_vector":
            return KeyVectorSparseAttention(d_model, n_heads, k, dropout, retrieval_config=rc)
        if kind == "routing":
            return RoutingSparseAttention(d_model, n_heads, router, k, dropout, layer_idx=layer,
                                          retrieval_config=rc)
        section = (config or {}).get("learned_address") or {}
        return LearnedAddressSparseAttention(
            d_model, n_heads, k, address_dim=section.get("address_dim", 32),
            similarity=section.get("similarity", "asymmetric"), dropout=dropout,
            address_module=self.address_book.get_address(layer) if self.address_book is not None else None,
            retrieval_config=rc)

    # ---- parameter groups (Phase A / Phase B training freezes one or the other)
    def get_router_parameters(self) -> list:
        return list(self.router.parameters()) if self.router is not None else []

    def get_address_parameters(self) -> list:
        if self.address_book is not None:
            return list(self.address_book.parameters())
        mods = [b.attn.address for b in self.blocks if hasattr(b.attn, "address")]
        return [p for m in mods for p in m.parameters()]

    @staticmethod
    def _set_trainable(params, flag: bool) -> None:
        for p in params:
            p.requires_grad_(flag)

    def freeze_router(self) -> None:
        self._set_trainable(self.get_router_parameters(), False)

    def unfreeze_router(self) -> None:
        self._set_trainable(self.get_router_parameters(), True)

    def freeze_addresses(self) -> None:
        self._set_trainable(self.get_address_parameters(), False)

    def unfreeze_addresses(self) -> None:
        self._set_trainable(self.get_address_parameters(), True)

    # ---- forward
    def _next_token_loss(self, logits: torch.Tensor, input_ids: torch.Tensor,
                         attn_mask: torch.Tensor) -> torch.Tensor:
        """Mean cross-entropy of positions 1..T-1 whose mask entry is set."""
        keep = attn_mask[:, 1:].bool()
        targets = input_ids[:, 1:].masked_fill(~keep, -100)
        total = F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]), targets.reshape(-1),
                                ignore_index=-100, reduction="sum")
        return total / keep.sum().clamp(min=1)

    def forward(
        self,
        input_ids: torch.Tensor,
        attn_mask: Optional[torch.Tensor] = None,
        labels: Optional[torch.Tensor] = None,
        question_index: Optional[torch.Tensor] = None,
        pointer_target_index: Optional[torch.Tensor] = None,
        pointer_target_slot: Optional[torch.Tensor] = None,
        return_hidden_states: bool = False,
        return_attentions: bool = False,
        return_per_head_attention: bool = False,
        return_pre_attention_hidden: bool = False,
        target_layer: Optional[int] = None,
        stop_after_layer: Optional[int] = None,
    ) -> dict[str, torch.Tensor]:
        """Token ids (B, T) -> {"logits", "loss"} plus what the return_* flags ask for.
        ``target_layer`` restricts attention / pre-attention capture (and the
        ``stop_after_layer`` check) to that layer."""
        del question_index, pointer_target_index, pointer_target_slot
        T = input_ids.shape[1]
        mask = attn_mask if attn_mask is not None else input_ids != self.pad_token_id
        x = self.dropout(self.token_emb(input_ids) + self.pos_emb.weight[:T].unsqueeze(0))
        caught = {"hidden_states": [], "attentions": [], "pre_attention_hidden": []}
        plain = not (return_hidden_states or return_attentions or return_pre_attention_hidden
                     or target_layer is not None or stop_after_layer is not None)
        if plain and not self.training and not torch.is_grad_enabled() and x.is_cuda:
            x = self._blocks_fused_norms(x, mask)
            return self._head(x, input_ids, mask, labels, caught, return_hidden_states,
                              return_attentions, return_pre_attention_hidden)
        for i, block in enumerate(self.blocks):
            watched = target_layer is None or i == target_layer
            if watched and return_pre_attention_hidden:
                caught["pre_attention_hidden"].append(block.ln1(x))
            if watched and return_attentions:
                x, w = block(x, attn_mask=mask, return_attention=True,
                             return_per_head=return_per_head_attention)
                caught["attentions"].append(w)
            else:
                x = block(x, attn_mask=mask)
            if return_hidden_states:
                caught["hidden_states"].append(x)
            if watched and stop_after_layer is not None and i >= stop_after_layer:
                break
        x = self.ln_f(x)
        return self._head(x, input_ids, mask, labels, caught, return_hidden_states,
                          return_attentions, return_pre_attention_hidden)

    @staticmethod
    def _add_norm(x: torch.Tensor, delta: torch.Tensor | None,
                  ln: nn.LayerNorm) -> tuple[torch.Tensor, torch.Tensor]:
        """(x + delta, ln(x + delta)) in one HIP pass where the kernel takes the shapes,
        else with the PyTorch ops (same values up to the norm's fp32 summation order)."""
        if _ln_kernel.supported(x, ln, delta):
            return _ln_kernel.residual_layer_norm(x, delta, ln)
        s = x if delta is None else x + delta
        return s, ln(s)

    def _blocks_fused_norms(self, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """Inference forward of the blocks and ln_f with every residual add fused into the
        LayerNorm that follows it: per block attn(ln1 x), then x += a with ln2 in one pass,
        ff(.), then x += f with the next block's ln1 (or ln_f) in one pass. Returns ln_f of
        the last residual stream. Dropout is the identity here (eval mode)."""
        blocks = list(self.blocks)
        x, h = self._add_norm(x, None, blocks[0].ln1)
        for i, block in enumerate(blocks):
            a = block.attn(h, attn_mask=mask)
            x, h = self._add_norm(x, a, block.ln2)
            f = block.ff(h)
            x, h = self._add_norm(x, f, blocks[i + 1].ln1 if i + 1 < len(blocks) else self.ln_f)
        return h

    def _head(self, x, input_ids, mask, labels, caught, return_hidden_states, return_attentions,
              return_pre_attention_hidden) -> dict[str, torch.Tensor]:
        """LM head, loss and the optional digit head over the final normalised stream x."""
        logits = self.lm_head(x)
        out: dict[str, torch.Tensor] = {"logits": logits,
                                        "loss": self._next_token_loss(logits, input_ids, mask)}
        if self.digit_head is not None and labels is not None:
            w = mask.to(x.dtype).unsqueeze(-1)
            pooled = (x * w).sum(dim=1) / w.sum(dim=1).clamp(min=1)
            digit_logits = self.digit_head(pooled)
            out["digit_loss"] = F.cross_entropy(digit_logits, labels)
            out["digit_accuracy"] = (digit_logits.argmax(dim=-1) == labels).float().mean()
        for flag, name in ((return_hidden_states, "hidden_states"), (return_attentions, "attentions"),
                           (return_pre_attention_hidden, "pre_attention_hidden")):
            if flag:
                out[name] = caught[name]
        return out
