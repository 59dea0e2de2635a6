"""Host-side behaviour of the drop-in Python API that needs no GPU: same names and
signatures as the reference, same error types, empty-selection semantics, no host
fallback, module state_dict keys."""

from __future__ import annotations

import inspect

import pytest
import torch

import routing_attention.kernels as K
from routing_attention.kernels import (
    SparseMeatConfig,
    causal_topk,
    fused_sparse_attention,
    sparse_meat_attention,
)
from routing_attention.models import LearnedAddressModule, LearnedAddressSparseAttention
from routing_attention.retrieval import RetrievalConfig, retrieval_config_from_dict


def test_public_names_match_reference():
    # reference routing_attention/kernels/__init__.py:23-31
    assert set(K.__all__) == {"causal_topk", "causal_topk_available", "causal_topk_reference",
                              "SparseMeatConfig", "sparse_meat_attention",
                              "fused_sparse_attention", "fused_sparse_attention_available"}


def test_signatures_match_reference():
    sig = inspect.signature(causal_topk)
    assert list(sig.parameters) == ["query", "key", "top_k", "method", "dtype", "prefer_triton"]
    assert sig.parameters["method"].default == "auto"
    sig = inspect.signature(sparse_meat_attention)
    assert list(sig.parameters) == ["q", "k", "v", "indices", "scale", "method", "config"]
    sig = inspect.signature(fused_sparse_attention)
    assert list(sig.parameters) == ["q_search", "k_search", "q", "k", "v", "top_k", "scale",
                                    "retrieval_method", "meat_method", "meat_config"]
    cfg = SparseMeatConfig()
    assert (cfg.method, cfg.block_d, cfg.k_pad, cfg.num_warps, cfg.compute_dtype) == \
        ("auto", None, None, 4, None)


def test_shape_errors_are_value_errors():
    with pytest.raises(ValueError, match="shape mismatch"):
        causal_topk(torch.zeros(1, 4, 8), torch.zeros(1, 5, 8), 2)
    with pytest.raises(ValueError, match="expected"):
        causal_topk(torch.zeros(4, 8), torch.zeros(4, 8), 2)


def test_empty_selection():
    out = causal_topk(torch.zeros(2, 5, 8), torch.zeros(2, 5, 8), 0)
    assert out.shape == (2, 5, 0) and out.dtype == torch.int32


def test_no_host_fallback():
    qa = torch.zeros(1, 16, 32)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        causal_topk(qa, qa, 4)
    q = torch.zeros(1, 2, 16, 32)
    idx = torch.zeros(1, 16, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        sparse_meat_attention(q, q, q, idx, 0.1)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        fused_sparse_attention(qa, qa, q, q, q, 4, 0.1)


def test_module_state_dict_keys_match_reference():
    m = LearnedAddressSparseAttention(d_model=256, n_heads=4, top_k=128, address_dim=32,
                                      retrieval_config={"use_fused_sparse": True})
    keys = set(m.state_dict())
    expect = {f"{p}.{w}" for p in ("q_proj", "k_proj", "v_proj", "out_proj",
                                   "address.q_addr_proj", "address.k_addr_proj")
              for w in ("weight", "bias")}
    assert keys == expect
    assert m.scale == 64 ** -0.5 and m._retrieval_cfg.use_fused_sparse


def test_retrieval_config_roundtrip():
    c = retrieval_config_from_dict({"use_fused_sparse": True, "method": "fused_causal", "top_k": 128})
    assert c.use_fused_sparse and c.method == "fused_causal" and c.top_k == 128
    assert c.dtype == RetrievalConfig().dtype == "float16"


def test_symmetric_address_module():
    m = LearnedAddressModule(64, 16, similarity="symmetric")
    x = torch.randn(2, 5, 64)
    q, k = m.forward_query_key(x)
    assert torch.equal(q, k) and torch.allclose(q.norm(dim=-1), torch.ones(2, 5))
