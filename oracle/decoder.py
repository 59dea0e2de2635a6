"""CPU restatement of the reference decoder around the sparse attention path.

TEST INFRASTRUCTURE ONLY (imported by tests/ and bench.py's CPU leg, never by the product).

It works from a ``state_dict`` and plain functional ops in float64, independent of the
product's module code, and follows the reference line by line:

* TransformerLM.forward, lm_token head and loss -- routing_attention/models/transformer.py
  :272-291 (embeddings), :299-330 (blocks), :332-333 (ln_f, tied lm_head), :361-373 (loss);
* TransformerBlock.forward -- transformer.py:50-73 (pre-norm, GELU MLP);
* the attention layers -- routing_attention/models/attention.py:
  learned_address :456-490 (LearnedAddressModule.forward_query_key,
  learned_address.py:39-46, for the search vectors), key_vector :361-393 with the search
  vectors of :339-341 *as called there* (query side = head-mean of K, key side = head-mean
  of Q), routing :577-606 (RouterMLP.forward_query_key, router.py:60-86).

Retrieval is the C oracle's exact causal top-K (``oracle.native``) on the float32-rounded
search vectors; the readout is the C oracle's double-accumulated softmax. ``forced_indices``
replaces the retrieval of each layer by given index tensors ("teacher forcing"): the
caller compares its own indices with the oracle's separately, and the rest of the forward
then runs on identical neighbour sets, so the outputs can be compared tightly.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle import native


def _lin(sd, name, x):
    w = sd[name + ".weight"]
    b = sd.get(name + ".bias")
    return F.linear(x, w, b)


def _ln(sd, name, x):
    d = x.shape[-1]
    return F.layer_norm(x, (d,), sd[name + ".weight"], sd[name + ".bias"], eps=1e-5)


def _mlp(sd, name, x):
    # nn.Sequential(Linear, GELU, Dropout, Linear[, Dropout]) in eval: indices 0 and 3
    return _lin(sd, name + ".3", F.gelu(_lin(sd, name + ".0", x)))


def search_vectors(sd, prefix, attention_type, x_norm, q, k, *, layer=0, normalize=True,
                   similarity="asymmetric"):
    """(query, key) search vectors of one layer, float64 (B, T, R)."""
    if attention_type == "learned_address":
        qa = _lin(sd, prefix + ".address.q_addr_proj", x_norm)
        ka = _lin(sd, prefix + ".address.k_addr_proj", x_norm) if similarity == "asymmetric" else qa
        if normalize:
            qa, ka = F.normalize(qa, dim=-1), F.normalize(ka, dim=-1)
        return qa, ka
    if attention_type == "key_vector":
        # attention.py:339-341 called as _search_vectors(q, k): returns (k.mean, q.mean)
        return k.mean(dim=1), q.mean(dim=1)
    if attention_type == "routing":
        # a single RouterMLP shared by the layers, or PerLayerRouter.routers[layer]
        r = prefix + ".router"
        if r + f".routers.{layer}.net.0.weight" in sd:
            r = r + f".routers.{layer}"
        qa = _mlp(sd, r + ".net", x_norm)
        ka = _mlp(sd, r + ".key_net", x_norm) if similarity == "asymmetric" else qa
        if normalize:
            qa, ka = F.normalize(qa, dim=-1), F.normalize(ka, dim=-1)
        return qa, ka
    raise ValueError(attention_type)


@torch.no_grad()
def decoder_forward(state_dict, input_ids, *, n_heads, top_k, attention_type="learned_address",
                    similarity="asymmetric", pad_token_id=0, forced_indices=None,
                    search_cast=None):
    """Logits (B, T, vocab) float64, loss, and per-layer oracle indices.

    ``search_cast``: dtype the product feeds its retrieval (e.g. bf16 for a bf16 model);
    the oracle's search vectors are rounded to it before the top-K.
    """
    sd = {k: v.detach().double().cpu() for k, v in state_dict.items()}
    n_layers = 1 + max(int(k.split(".")[1]) for k in sd if k.startswith("blocks."))
    ids = input_ids.cpu()
    B, T = ids.shape
    x = sd["token_emb.weight"][ids] + sd["pos_emb.weight"][:T].unsqueeze(0)
    layer_idx_out = []
    for li in range(n_layers):
        p = f"blocks.{li}"
        xn = _ln(sd, p + ".ln1", x)
        d_model = xn.shape[-1]
        hd = d_model // n_heads
        q = _lin(sd, p + ".attn.q_proj", xn).view(B, T, n_heads, hd).transpose(1, 2)
        k = _lin(sd, p + ".attn.k_proj", xn).view(B, T, n_heads, hd).transpose(1, 2)
        v = _lin(sd, p + ".attn.v_proj", xn).view(B, T, n_heads, hd).transpose(1, 2)
        qs, ks = search_vectors(sd, p + ".attn", attention_type, xn, q, k, layer=li,
                                similarity=similarity)
        if search_cast is not None:
            qs, ks = qs.to(search_cast), ks.to(search_cast)
        idx = native.causal_topk(qs.float(), ks.float(), top_k)
        layer_idx_out.append(idx)
        use = forced_indices[li].cpu() if forced_indices is not None else idx
        meat = native.sparse_readout(q.float(), k.float(), v.float(), use, hd ** -0.5)
        attn = _lin(sd, p + ".attn.out_proj", meat.transpose(1, 2).reshape(B, T, d_model))
        x = x + attn
        x = x + _mlp(sd, p + ".ff", _ln(sd, p + ".ln2", x))
    x = _ln(sd, "ln_f", x)
    logits = F.linear(x, sd["token_emb.weight"])   # lm_head tied to token_emb
    mask = (ids != pad_token_id)[:, 1:].double()
    ce = F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]), ids[:, 1:].reshape(-1),
                         reduction="none").view(B, T - 1)
    loss = (ce * mask).sum() / mask.sum().clamp(min=1)
    return logits, loss, layer_idx_out
