"""Decoder-only language model around the sparse attention modules (mirrors
routing_attention/models/transformer.py of the reference: TransformerBlock (:26-73) and
TransformerLM (:76-401) with the same constructor, submodule names, state_dict keys, weight
tying and loss).

Attention types on the MI355X path: ``learned_address``, ``key_vector``, ``routing`` (the
top-K sparse modules, HIP retrieval + readout) and ``dense`` / ``dense_flash``
(F.scaled_dot_product_attention, the comparator). ``linear`` and ``local`` attention and
the pointer / pool output heads are not part of this build and raise.
"""

from __future__ import annotations

from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from routing_attention.models.attention import (
    DenseSDPAAttention,
    KeyVectorSparseAttention,
    LearnedAddressSparseAttention,
    RoutingSparseAttention,
)
from routing_attention.models.learned_address import build_address_book_from_config
from routing_attention.models.router import RouterMLP, build_router_from_config

_OUT_OF_SCOPE_ATTENTION = ("linear", "local")


class TransformerBlock(nn.Module):
    """Pre-norm block: x + attn(ln1(x)), then x + ff(ln2(x)) (reference :26-73)."""

    def __init__(self, d_model: int, n_heads: int, d_ff: int, dropout: float,
                 attention_module: nn.Module, layer_idx: int = 0):
        super().__init__()
        self.attn = attention_module
        self.layer_idx = layer_idx
        self.ln1 = nn.LayerNorm(d_model)
        self.ln2 = nn.LayerNorm(d_model)
        self.ff = nn.Sequential(
            nn.Linear(d_model, d_ff),
            nn.GELU(),
            nn.Dropout(dropout),
            nn.Linear(d_ff, d_model),
            nn.Dropout(dropout),
        )

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_attention: bool = False, return_per_head: bool = False, **attn_kwargs):
        residual = x
        x_norm = self.ln1(x)
        if return_attention:
            attn_out, attn_w = self.attn(x_norm, attn_mask=attn_mask, return_attention=True,
                                         return_per_head=return_per_head, **attn_kwargs)
            x = residual + attn_out
            x = x + self.ff(self.ln2(x))
            return x, attn_w
        x = residual + self.attn(x_norm, attn_mask=attn_mask, **attn_kwargs)
        return x + self.ff(self.ln2(x))


class TransformerLM(nn.Module):
    """Decoder-only transformer for language modelling (reference :76-401)."""

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
        if attention_type in _OUT_OF_SCOPE_ATTENTION:
            raise NotImplementedError(f"attention_type={attention_type!r} is not part of this build")
        self.d_model = d_model
        self.output_head = output_head
        self.pointer_target_mode = pointer_target_mode
        self.max_seq_len = max_seq_len
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.pad_token_id = pad_token_id
        self.attention_type = attention_type
        self.routing_top_k = routing_top_k
        self.retrieval_config = retrieval_config
        if retrieval_config is None and config is not None:
            self.retrieval_config = config.get("retrieval")
        if router is None and attention_type == "routing" and config is not None:
            router = build_router_from_config(config)
        self.router = router
        self.address_book = None
        la_cfg = (config or {}).get("learned_address", {})

        self.token_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Embedding(max_seq_len, d_model)
        self.dropout = nn.Dropout(dropout)

        self.blocks = nn.ModuleList()
        for layer_idx in range(n_layers):
            if attention_type in ("dense", "dense_flash"):
                attn = DenseSDPAAttention(d_model, n_heads, dropout)
            elif attention_type == "key_vector":
                attn = KeyVectorSparseAttention(d_model, n_heads, routing_top_k, dropout,
                                                retrieval_config=self.retrieval_config)
            elif attention_type == "learned_address":
                if self.address_book is None and config is not None:
                    self.address_book = build_address_book_from_config(config)
                addr_mod = (self.address_book.get_address(layer_idx)
                            if self.address_book is not None else None)
                attn = LearnedAddressSparseAttention(
                    d_model, n_heads, routing_top_k,
                    address_dim=la_cfg.get("address_dim", 32),
                    similarity=la_cfg.get("similarity", "asymmetric"),
                    dropout=dropout, address_module=addr_mod,
                    retrieval_config=self.retrieval_config,
                )
            elif attention_type == "routing":
                if router is None:
                    router = RouterMLP(d_model, routing_dim=32)
                attn = RoutingSparseAttention(d_model, n_heads, router, routing_top_k, dropout,
                                              layer_idx=layer_idx,
                                              retrieval_config=self.retrieval_config)
            else:
                raise ValueError(f"Unknown attention_type: {attention_type}")
            self.blocks.append(TransformerBlock(d_model, n_heads, d_ff, dropout, attn, layer_idx=layer_idx))

        self.ln_f = nn.LayerNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.token_emb.weight
        self.num_digit_classes = num_digit_classes
        self.digit_head = nn.Linear(d_model, num_digit_classes) if num_digit_classes > 0 else None

    def get_router_parameters(self):
        return [] if self.router is None else list(self.router.parameters())

    def get_address_parameters(self):
        if self.address_book is not None:
            return list(self.address_book.parameters())
        params = []
        for block in self.blocks:
            if hasattr(block.attn, "address"):
                params.extend(block.attn.address.parameters())
        return params

    def freeze_router(self) -> None:
        for p in self.get_router_parameters():
            p.requires_grad = False

    def unfreeze_router(self) -> None:
        for p in self.get_router_parameters():
            p.requires_grad = True

    def freeze_addresses(self) -> None:
        for p in self.get_address_parameters():
            p.requires_grad = False

    def unfreeze_addresses(self) -> None:
        for p in self.get_address_parameters():
            p.requires_grad = True

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
        """Token ids (B, T) -> {"logits", "loss", ...} (reference :272-401, lm_token head)."""
        del question_index, pointer_target_index, pointer_target_slot
        B, T = input_ids.shape
        if attn_mask is None:
            attn_mask = input_ids != self.pad_token_id
        pos = torch.arange(T, device=input_ids.device).unsqueeze(0)
        x = self.dropout(self.token_emb(input_ids) + self.pos_emb(pos))

        hidden_states, pre_attention_hidden, attentions = [], [], []
        for layer_idx, block in enumerate(self.blocks):
            if target_layer is not None and layer_idx != target_layer:
                x = block(x, attn_mask=attn_mask)
                if return_hidden_states:
                    hidden_states.append(x)
                continue
            if return_pre_attention_hidden:
                pre_attention_hidden.append(block.ln1(x))
            if return_attentions:
                x, attn_w = block(x, attn_mask=attn_mask, return_attention=True,
                                  return_per_head=return_per_head_attention)
                attentions.append(attn_w)
            else:
                x = block(x, attn_mask=attn_mask)
            if return_hidden_states:
                hidden_states.append(x)
            if stop_after_layer is not None and layer_idx >= stop_after_layer:
                break

        x = self.ln_f(x)
        logits = self.lm_head(x)
        output: dict[str, torch.Tensor] = {"logits": logits}

        # next-token loss over non-pad targets (reference :361-373)
        shift_logits = logits[:, :-1, :].contiguous()
        shift_labels = input_ids[:, 1:].contiguous()
        shift_mask = attn_mask[:, 1:].contiguous().float()
        loss = F.cross_entropy(shift_logits.view(-1, shift_logits.size(-1)), shift_labels.view(-1),
                               reduction="none").view(B, T - 1)
        output["loss"] = (loss * shift_mask).sum() / shift_mask.sum().clamp(min=1)
        if self.digit_head is not None and labels is not None:
            mask = attn_mask.float()
            pooled = (x * mask.unsqueeze(-1)).sum(dim=1) / mask.sum(dim=1, keepdim=True).clamp(min=1)
            digit_logits = self.digit_head(pooled)
            output["digit_loss"] = F.cross_entropy(digit_logits, labels)
            output["digit_accuracy"] = (digit_logits.argmax(dim=-1) == labels).float().mean()
        if return_hidden_states:
            output["hidden_states"] = hidden_states
        if return_pre_attention_hidden:
            output["pre_attention_hidden"] = pre_attention_hidden
        if return_attentions:
            output["attentions"] = attentions
        return output
