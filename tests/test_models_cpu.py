"""Host-side checks of the model layer that need no GPU: reference names, constructor
defaults and state_dict keys of the sparse modules, the decoder and the routers; the
vectorised candidate merge against the reference's per-row loop; the decoder oracle's
teacher forcing; out-of-scope options raising."""

from __future__ import annotations

import inspect

import pytest
import torch

from routing_attention.models import (
    KeyVectorSparseAttention,
    LearnedAddressSparseAttention,
    MultiScaleRouter,
    PerLayerAddressBook,
    PerLayerRouter,
    RouterMLP,
    RoutingSparseAttention,
    TransformerLM,
    build_address_book_from_config,
    build_router_from_config,
)
from routing_attention.models.router import merge_candidate_sets


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


def test_router_config_factory():
    cfg = {"model": {"d_model": 64, "n_layers": 3, "n_heads": 4}, "router": {}}
    r = build_router_from_config(cfg)
    assert isinstance(r, PerLayerRouter) and len(r.routers) == 3
    cfg["router"] = {"mode": "single", "loss_type": "mse", "routing_dim": 16}
    r = build_router_from_config(cfg)
    assert isinstance(r, RouterMLP) and not r.normalize and r.use_affine_dot
    cfg["router"] = {"mode": "multi_scale"}
    assert isinstance(build_router_from_config(cfg), MultiScaleRouter)
    book = build_address_book_from_config({"model": {"d_model": 64, "n_layers": 2},
                                           "learned_address": {"address_dim": 16}})
    assert isinstance(book, PerLayerAddressBook) and book.get_address(1).address_dim == 16


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


def _merge_loop(a, b, k):
    # the per-row loop of reference router.py:195-204, restated
    B, T, _ = a.shape
    out = torch.zeros(B, T, k, dtype=torch.long)
    for bb in range(B):
        for i in range(T):
            cand = torch.cat([a[bb, i], b[bb, i]]).unique()
            n = min(k, cand.numel())
            out[bb, i, :n] = cand[:n]
            if n < k:
                out[bb, i, n:] = cand[0]
    return out


@pytest.mark.parametrize("ka,kb,k,hi", [(4, 4, 8, 6), (4, 4, 8, 50), (3, 5, 8, 4), (1, 1, 2, 3), (8, 8, 10, 9)])
def test_merge_candidate_sets_matches_reference_loop(ka, kb, k, hi):
    g = torch.Generator().manual_seed(ka * 100 + kb * 10 + hi)
    a = torch.randint(0, hi, (2, 7, ka), generator=g)
    b = torch.randint(0, hi, (2, 7, kb), generator=g)
    assert torch.equal(merge_candidate_sets(a, b, k), _merge_loop(a, b, k))


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
