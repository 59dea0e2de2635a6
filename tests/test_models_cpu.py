"""Host-side checks of the model layer that need no GPU: reference names, constructor
defaults and state_dict keys of the sparse modules, the decoder and the router; the
decoder's loss and capture options; the decoder oracle's teacher forcing; out-of-scope
options raising."""

from __future__ import annotations

import inspect

import pytest
import torch

from routing_attention.models import (
    KeyVectorSparseAttention,
    LearnedAddressSparseAttention,
    PerLayerAddressBook,
    RouterMLP,
    RoutingSparseAttention,
    TransformerLM,
    build_address_book_from_config,
)


def _keys(m):
    return sorted(m.state_dict().keys())


def test_sparse_module_state_dict_keys():
    # key names of reference attention.py:324-334, 421-439, 526-545 and router.py:41-58
    proj = ["k_proj.bias", "k_proj.weight", "out_proj.bias", "out_proj.weight", "q_proj.bias",
            "q_proj.weight", "v_proj.bias", "v_proj.weight"]
    assert _keys(KeyVectorSparseAttention(64, 4, 8)) == proj
    la = _keys(LearnedAddressSparseAttention(64, 4, 8))
    assert la == sorted(proj + ["address.q_addr_proj.weight", "address.q_addr_proj.bias",
                                "address.k_addr_proj.weight", "address.k_addr_proj.bias"])
    r = RouterMLP(64, 32, similarity="asymmetric")
    assert _keys(r) == sorted(f"{n}.{i}.{p}" for n in ("net", "key_net") for i in (0, 3)
                              for p in ("weight", "bias"))
    assert r.net[0].out_features == max(32 * 2, 64 // 4)   # reference hidden_dim default
    rs = _keys(RoutingSparseAttention(64, 4, RouterMLP(64, 16), 8))
    assert rs == sorted(proj + [f"router.net.{i}.{p}" for i in (0, 3) for p in ("weight", "bias")])


def test_address_book_config_and_router_modes():
    book = build_address_book_from_config({"model": {"d_model": 64, "n_layers": 2},
                                           "learned_address": {"address_dim": 16}})
    assert isinstance(book, PerLayerAddressBook) and book.get_address(1).address_dim == 16
    assert book.get_router(0) is book.get_address(0)
    alias = build_address_book_from_config({"model": {"d_model": 64, "n_layers": 1},
                                            "learned_address": {"routing_dim": 8, "similarity": "symmetric"}})
    assert alias.get_address(0).address_dim == 8 and alias.get_address(0).k_addr_proj is None
    # a config asking for the reference's per-layer / multi-scale routers raises; single works
    cfg = {"model": {"d_model": 64, "n_layers": 2}, "router": {}}
    with pytest.raises(NotImplementedError):
        TransformerLM(16, 64, 2, 4, 64, 16, attention_type="routing", config=cfg)
    cfg["router"] = {"mode": "single", "routing_dim": 16, "similarity": "asymmetric"}
    m = TransformerLM(16, 64, 2, 4, 64, 16, attention_type="routing", config=cfg)
    assert isinstance(m.router, RouterMLP) and m.blocks[1].attn.router is m.router
    assert m.router.routing_dim == 16 and hasattr(m.router, "key_net")
    assert any(k.startswith("router.net.") for k in m.state_dict())


def test_router_forward_shapes_and_normalisation():
    torch.manual_seed(0)
    x = torch.randn(2, 10, 64)
    r = RouterMLP(64, 16, similarity="asymmetric", n_heads=4, per_head_routing=True)
    q, k = r.forward_query_key(x)
    assert q.shape == (2, 10, 4, 16) and not torch.equal(q, k)
    torch.testing.assert_close(q.norm(dim=-1), torch.ones(2, 10, 4))
    s = r.retrieval_scores(x)
    ref = torch.einsum("bthq,bshq->bts", q, k) / 4          # reference router.py:112-113
    torch.testing.assert_close(s, ref)
    p = r.pairwise_scores(q, k)
    torch.testing.assert_close(p, torch.einsum("bthq,bshq->bhts", q, k).mean(dim=2))


def test_router_affine_and_symmetric():
    torch.manual_seed(1)
    x = torch.randn(2, 12, 32)
    r = RouterMLP(32, 8, normalize=False, use_affine_dot=True)
    q, k = r.forward_query_key(x)
    assert q is k and q.shape == (2, 12, 8)
    with torch.no_grad():
        r.dot_scale.fill_(2.0)
        r.dot_bias.fill_(-1.0)
    torch.testing.assert_close(r.pairwise_scores(q), 2.0 * (q @ q.transpose(1, 2)) - 1.0)
    assert sorted(r.state_dict()) == sorted(["dot_bias", "dot_scale", "net.0.bias", "net.0.weight",
                                             "net.3.bias", "net.3.weight"])


def test_decoder_loss_and_capture_options():
    """The masked next-token loss equals the per-token cross-entropy averaged over the
    unmasked targets; hidden states / pre-attention captures and stop_after_layer."""
    torch.manual_seed(2)
    m = TransformerLM(20, 32, 3, 2, 64, 16, dropout=0.0, attention_type="dense").eval()
    ids = torch.randint(1, 20, (2, 16))
    ids[1, 10:] = 0   # padding (pad_token_id 0) in the second sequence
    out = m(ids, return_hidden_states=True, return_pre_attention_hidden=True)
    logits = out["logits"]
    ce = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, 20), ids[:, 1:].reshape(-1),
                                           reduction="none").view(2, 15)
    w = (ids[:, 1:] != 0).float()
    torch.testing.assert_close(out["loss"], (ce * w).sum() / w.sum())
    assert len(out["hidden_states"]) == 3 and len(out["pre_attention_hidden"]) == 3
    torch.testing.assert_close(out["pre_attention_hidden"][1], m.blocks[1].ln1(out["hidden_states"][0]))
    short = m(ids, return_hidden_states=True, stop_after_layer=0)
    assert len(short["hidden_states"]) == 1
    only = m(ids, return_pre_attention_hidden=True, target_layer=2)
    assert len(only["pre_attention_hidden"]) == 1


def test_decoder_signature_and_scope():
    sig = inspect.signature(TransformerLM.__init__)
    names = list(sig.parameters)[1:]
    assert names[:8] == ["vocab_size", "d_model", "n_layers", "n_heads", "d_ff", "max_seq_len",
                         "dropout", "attention_type"]
    assert sig.parameters["routing_top_k"].default == 32
    with pytest.raises(NotImplementedError):
        TransformerLM(16, 32, 1, 2, 64, 16, attention_type="linear")
    with pytest.raises(NotImplementedError):
        TransformerLM(16, 32, 1, 2, 64, 16, output_head="pointer_mlp")
    with pytest.raises(ValueError, match="Unknown attention_type"):
        TransformerLM(16, 32, 1, 2, 64, 16, attention_type="nope")


def test_decoder_state_dict_and_tying():
    m = TransformerLM(128, 64, 2, 4, 256, 32, attention_type="learned_address", routing_top_k=8,
                      config={"model": {"d_model": 64, "n_layers": 2},
                              "learned_address": {"address_dim": 16}})
    keys = set(m.state_dict().keys())
    # tied head (reference transformer.py:189), per-layer address book (:155-160)
    assert m.lm_head.weight is m.token_emb.weight
    assert "address_book.addresses.1.q_addr_proj.weight" in keys
    assert "blocks.1.attn.address.k_addr_proj.weight" in keys
    assert {"blocks.0.ff.0.weight", "blocks.0.ff.3.weight", "ln_f.weight", "pos_emb.weight"} <= keys
    assert m.blocks[1].attn.address is m.address_book.get_address(1)
    r = TransformerLM(128, 64, 2, 4, 256, 32, attention_type="routing")
    assert r.blocks[0].attn.router is r.blocks[1].attn.router     # one shared RouterMLP
    assert r.router is None and not any(k.startswith("router.") for k in r.state_dict())


def test_decoder_oracle_teacher_forcing_and_self_indices():
    """oracle.decoder: with forced indices equal to its own, the forward is unchanged; with
    every row forced onto itself, attention reduces to v_t (softmax over K copies)."""
    from oracle.decoder import decoder_forward

    torch.manual_seed(3)
    m = TransformerLM(32, 32, 2, 2, 64, 64, dropout=0.0, attention_type="learned_address",
                      routing_top_k=8)
    sd = m.state_dict()
    ids = torch.randint(0, 32, (2, 40), generator=torch.Generator().manual_seed(4))
    logits, loss, idx = decoder_forward(sd, ids, n_heads=2, top_k=8)
    logits2, loss2, _ = decoder_forward(sd, ids, n_heads=2, top_k=8, forced_indices=idx)
    assert torch.equal(logits, logits2) and torch.isfinite(loss)
    # rows forced onto themselves: the block is x + out_proj(v(ln1(x))) + ff
    B, T = ids.shape
    self_idx = [torch.arange(T).view(1, T, 1).expand(B, T, 8).to(torch.int32)] * 2
    got, _, _ = decoder_forward(sd, ids, n_heads=2, top_k=8, forced_indices=self_idx)
    sdd = {k: v.double() for k, v in sd.items()}
    x = sdd["token_emb.weight"][ids] + sdd["pos_emb.weight"][:T]
    for li in range(2):
        p = f"blocks.{li}"
        ln = lambda n, y: torch.nn.functional.layer_norm(y, (32,), sdd[n + ".weight"], sdd[n + ".bias"])
        lin = lambda n, y: y @ sdd[n + ".weight"].T + sdd[n + ".bias"]
        x = x + lin(p + ".attn.out_proj", lin(p + ".attn.v_proj", ln(p + ".ln1", x)))
        x = x + lin(p + ".ff.3", torch.nn.functional.gelu(lin(p + ".ff.0", ln(p + ".ln2", x))))
    x = torch.nn.functional.layer_norm(x, (32,), sdd["ln_f.weight"], sdd["ln_f.bias"])
    # the oracle's readout takes q/k/v rounded to float32: 1e-7-level differences
    torch.testing.assert_close(got, x @ sdd["token_emb.weight"].T, rtol=1e-5, atol=1e-5)
