"""C-ABI checks that need no GPU: the library loads, exports every symbol the public header
declares, and reports contract violations as status codes before any HIP call."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from routing_attention.kernels import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "wayfinder_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(wf_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_the_abi():
    names = _declared()
    assert names == sorted(_lib.SIGNATURES), names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.wf_abi_version() == _lib.ABI_VERSION == 5


def _i64(*v):
    return (ctypes.c_int64 * len(v))(*v)


FAKE = 0x1000  # never dereferenced: every call below fails validation first


def _topk(lib, **kw):
    a = dict(query=FAKE, key=FAKE, dtype=2, B=1, T=64, R=32, qs=_i64(64 * 32, 32, 1),
             ks=_i64(64 * 32, 32, 1), top_k=8, out=FAKE, scores=None, ws=FAKE, ws_bytes=1 << 20)
    a.update(kw)
    return lib.wf_causal_topk_fwd(a["query"], a["key"], a["dtype"], a["B"], a["T"], a["R"],
                                  a["qs"], a["ks"], a["top_k"], a["out"], a["scores"], a["ws"],
                                  a["ws_bytes"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=9), _lib.WF_ERR_UNSUPPORTED, "dtype"),
    (dict(R=0), _lib.WF_ERR_INVALID_ARGUMENT, "shape"),
    (dict(T=-1), _lib.WF_ERR_INVALID_ARGUMENT, "shape"),
    (dict(top_k=-3), _lib.WF_ERR_INVALID_ARGUMENT, "top_k"),
    (dict(R=257), _lib.WF_ERR_UNSUPPORTED, "R=257"),
    (dict(top_k=600, T=1000), _lib.WF_ERR_UNSUPPORTED, "k_eff"),
    (dict(query=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(out=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(qs=None), _lib.WF_ERR_INVALID_ARGUMENT, "stride"),
    (dict(ws=None), _lib.WF_ERR_WORKSPACE, "workspace"),
    (dict(ws_bytes=4), _lib.WF_ERR_WORKSPACE, "workspace"),
])
def test_topk_contract_errors(lib, kw, code, msg):
    assert _topk(lib, **kw) == code
    assert msg in _lib.last_error()


def test_topk_empty_problems_are_noops(lib):
    assert _topk(lib, B=0) == _lib.WF_OK
    assert _topk(lib, top_k=0) == _lib.WF_OK
    assert _topk(lib, T=0) == _lib.WF_OK
    assert _lib.last_error() == ""


def test_workspace_size(lib):
    assert lib.wf_causal_topk_workspace_bytes(1, 16384, 32, 128) == 256
    assert lib.wf_causal_topk_workspace_bytes(4, 65536, 32, 256) == 4 * 256 * 4
    assert lib.wf_causal_topk_workspace_bytes(0, 10, 32, 8) == 0
    assert lib.wf_fused_workspace_bytes(2, 1000, 32, 8) == lib.wf_causal_topk_workspace_bytes(2, 1000, 32, 8)
    # backward workspace: a pure function of the shape (no device query): offsets, two
    # ping-pong (key, row) arrays, row stats, radix histograms (256 per 4096-slot tile), totals
    a256 = lambda x: (x + 255) // 256 * 256
    for B, H, T, K in ((1, 8, 16384, 128), (2, 3, 300, 7)):
        n = B * T * K
        want = (a256((B * T + 1) * 4) + 4 * a256(n * 4) + a256(B * H * T * 8)
                + a256(256 * ((n + 4095) // 4096) * 4) + a256(256 * 4))
        assert lib.wf_sparse_readout_bwd_workspace_bytes(B, H, T, K) == want
    assert lib.wf_sparse_readout_bwd_workspace_bytes(1, 1, 0, 4) == 0


def _readout(lib, **kw):
    s4 = _i64(8 * 64 * 64, 64 * 64, 64, 1)
    a = dict(q=FAKE, k=FAKE, v=FAKE, dtype=2, B=1, H=8, T=64, D=64, qs=s4, ks=s4, vs=s4,
             idx=FAKE, is_=_i64(64 * 8, 8, 1), K=8, scale=0.125, flags=0, out=FAKE, os=s4)
    a.update(kw)
    return lib.wf_sparse_readout_fwd(a["q"], a["k"], a["v"], a["dtype"], a["B"], a["H"], a["T"],
                                     a["D"], a["qs"], a["ks"], a["vs"], a["idx"], a["is_"], a["K"],
                                     a["scale"], a["flags"], a["out"], a["os"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=-1), _lib.WF_ERR_UNSUPPORTED, "dtype"),
    (dict(D=300), _lib.WF_ERR_UNSUPPORTED, "head_dim"),
    (dict(K=0), _lib.WF_ERR_INVALID_ARGUMENT, "K must"),
    (dict(K=5000), _lib.WF_ERR_UNSUPPORTED, "K=5000"),
    (dict(H=-2), _lib.WF_ERR_INVALID_ARGUMENT, "shape"),
    (dict(v=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(idx=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(os=None), _lib.WF_ERR_INVALID_ARGUMENT, "stride"),
])
def test_readout_contract_errors(lib, kw, code, msg):
    assert _readout(lib, **kw) == code
    assert msg in _lib.last_error()


def test_readout_empty_is_noop(lib):
    assert _readout(lib, T=0) == _lib.WF_OK


def test_fused_contract_errors(lib):
    assert lib.wf_fused_topk_sparse_fwd(None, None) == _lib.WF_ERR_INVALID_ARGUMENT
    a = _lib.FusedArgs()
    a.q_search = a.k_search = a.q = a.k = a.v = a.out = a.out_idx = FAKE
    a.workspace, a.workspace_bytes = FAKE, 1 << 20
    a.qs_strides[:] = [64 * 32, 32, 1]
    a.ks_strides[:] = [64 * 32, 32, 1]
    for f in ("q_strides", "k_strides", "v_strides", "out_strides"):
        getattr(a, f)[:] = [8 * 64 * 64, 64 * 64, 64, 1]
    a.B, a.H, a.T, a.D, a.R, a.top_k = 1, 8, 64, 64, 32, 8
    a.search_dtype, a.dtype, a.scale = 2, 2, 0.125
    a.D = 300
    assert lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), None) == _lib.WF_ERR_UNSUPPORTED
    a.D, a.top_k = 64, 0
    assert lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), None) == _lib.WF_ERR_INVALID_ARGUMENT
    a.top_k, a.workspace_bytes = 8, 0
    assert lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), None) == _lib.WF_ERR_WORKSPACE


def test_status_maps_to_reference_exception_types():
    with pytest.raises(ValueError):
        _lib.check(_lib.WF_ERR_INVALID_ARGUMENT)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.WF_ERR_UNSUPPORTED)
    with pytest.raises(_lib.WayfinderHipError):
        _lib.check(_lib.WF_ERR_HIP)
    _lib.check(_lib.WF_OK)


def _bwd(lib, **kw):
    B, H, T, D, K = 1, 2, 64, 64, 8
    st = (H * T * D, D, H * D, 1)          # (B, T, H, D) memory viewed as (B, H, T, D)
    a = _lib.ReadoutBwdArgs()
    a.q = a.k = a.v = a.dout = a.dq = a.dk = a.dv = FAKE
    a.indices = a.lse2 = a.workspace = FAKE
    a.workspace_bytes = 1 << 30
    for f in ("q", "k", "v", "dout", "dq", "dk", "dv"):
        getattr(a, f + "_strides")[:] = list(st)
    a.idx_strides[:] = [T * K, K, 1]
    a.B, a.H, a.T, a.D, a.K = B, H, T, D, K
    a.dtype, a.scale, a.flags = 2, 0.125, 0
    for k, v in kw.items():
        if k.endswith("_strides"):
            getattr(a, k)[:] = list(v)
        else:
            setattr(a, k, v)
    return lib.wf_sparse_readout_bwd(ctypes.byref(a), None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=7), _lib.WF_ERR_UNSUPPORTED, "dtype"),
    (dict(D=300), _lib.WF_ERR_UNSUPPORTED, "head_dim"),
    (dict(K=0), _lib.WF_ERR_INVALID_ARGUMENT, "K must be"),
    (dict(K=2000), _lib.WF_ERR_UNSUPPORTED, "K=2000"),
    (dict(dout=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(dk=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(lse2=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(q_strides=(2 * 64 * 64, 64, 128, 2)), _lib.WF_ERR_UNSUPPORTED, "contiguous head dim"),
    (dict(dv=FAKE + 2), _lib.WF_ERR_UNSUPPORTED, "16-byte"),
    (dict(idx_strides=(64 * 8, 8, 2)), _lib.WF_ERR_UNSUPPORTED, "index rows"),
])
def test_readout_bwd_contract_errors(lib, kw, code, msg):
    assert _bwd(lib, **kw) == code
    assert msg in _lib.last_error()


def test_readout_bwd_empty_is_noop(lib):
    assert _bwd(lib, T=0) == _lib.WF_OK
    assert _bwd(lib, B=0) == _lib.WF_OK


@pytest.mark.parametrize("p", [-0.1, 1.0, 1.5, float("nan")])
def test_dropout_probability_contract(lib, p):
    st = _i64(2 * 64 * 64, 64, 128, 1)
    rc = lib.wf_sparse_readout_fwd_dropout(FAKE, FAKE, FAKE, 2, 1, 2, 64, 64, st, st, st, FAKE,
                                           _i64(64 * 8, 8, 1), 8, 0.125, 0, p, 1, FAKE, st, FAKE, None)
    assert rc == _lib.WF_ERR_INVALID_ARGUMENT and "dropout_p" in _lib.last_error()
    a = _lib.ReadoutBwdArgs()
    assert lib.wf_sparse_readout_bwd_dropout(ctypes.byref(a), p, 1, None) == _lib.WF_ERR_INVALID_ARGUMENT
    assert "dropout_p" in _lib.last_error()


def test_dropout_forward_needs_lse(lib):
    st = _i64(2 * 64 * 64, 64, 128, 1)
    rc = lib.wf_sparse_readout_fwd_dropout(FAKE, FAKE, FAKE, 2, 1, 2, 64, 64, st, st, st, FAKE,
                                           _i64(64 * 8, 8, 1), 8, 0.125, 0, 0.1, 1, FAKE, st, None, None)
    assert rc == _lib.WF_ERR_INVALID_ARGUMENT and "lse2" in _lib.last_error()


def test_readout_fwd_lse_needs_lse(lib):
    st = _i64(2 * 64 * 64, 64, 128, 1)
    rc = lib.wf_sparse_readout_fwd_lse(FAKE, FAKE, FAKE, 2, 1, 2, 64, 64, st, st, st, FAKE,
                                       _i64(64 * 8, 8, 1), 8, 0.125, 0, FAKE, st, None, None)
    assert rc == _lib.WF_ERR_INVALID_ARGUMENT and "lse2" in _lib.last_error()


def _addr(lib, **kw):
    a = dict(x=FAKE, dtype=2, B=1, T=16, D=64, xs=_i64(16 * 64, 64, 1), wq=FAKE, bq=None, wk=FAKE,
             bk=None, ws=64, R=32, norm=1, oq=FAKE, oqs=_i64(16 * 32, 32, 1), ok=FAKE,
             oks=_i64(16 * 32, 32, 1))
    a.update(kw)
    return lib.wf_address_project_fwd(a["x"], a["dtype"], a["B"], a["T"], a["D"], a["xs"], a["wq"],
                                      a["bq"], a["wk"], a["bk"], a["ws"], a["R"], a["norm"], a["oq"],
                                      a["oqs"], a["ok"], a["oks"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=5), _lib.WF_ERR_UNSUPPORTED, "dtype"),
    (dict(R=33), _lib.WF_ERR_UNSUPPORTED, "R=33"),
    (dict(D=60, ws=60), _lib.WF_ERR_UNSUPPORTED, "multiple of 8"),
    (dict(R=0), _lib.WF_ERR_INVALID_ARGUMENT, "shape"),
    (dict(x=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(ok=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(xs=_i64(16 * 64, 64, 2)), _lib.WF_ERR_UNSUPPORTED, "contiguous last dim"),
    (dict(wq=FAKE + 4), _lib.WF_ERR_UNSUPPORTED, "16-byte"),
    (dict(oks=None), _lib.WF_ERR_INVALID_ARGUMENT, "stride"),
])
def test_address_contract_errors(lib, kw, code, msg):
    assert _addr(lib, **kw) == code
    assert msg in _lib.last_error()


def test_address_empty_is_noop(lib):
    assert _addr(lib, B=0) == _lib.WF_OK


def _ln(lib, **kw):
    a = dict(x=FAKE, d=FAKE, dtype=2, rows=16, n=256, xs=256, ds=256, w=FAKE, b=FAKE, eps=1e-5,
             s=FAKE, ss=256, y=FAKE, ys=256)
    a.update(kw)
    return lib.wf_residual_layernorm_fwd(a["x"], a["d"], a["dtype"], a["rows"], a["n"], a["xs"], a["ds"],
                                         a["w"], a["b"], a["eps"], a["s"], a["ss"], a["y"], a["ys"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dtype=7), _lib.WF_ERR_UNSUPPORTED, "dtype"),
    (dict(n=260, xs=264, ds=264, ss=264, ys=264), _lib.WF_ERR_UNSUPPORTED, "multiple of 8"),
    (dict(n=1032, xs=1032, ds=1032, ss=1032, ys=1032), _lib.WF_ERR_UNSUPPORTED, "at most 1024"),
    (dict(rows=-1), _lib.WF_ERR_INVALID_ARGUMENT, "shape"),
    (dict(eps=-1.0), _lib.WF_ERR_INVALID_ARGUMENT, "eps"),
    (dict(y=None), _lib.WF_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(xs=128), _lib.WF_ERR_UNSUPPORTED, "strides"),
    (dict(d=FAKE + 2), _lib.WF_ERR_UNSUPPORTED, "alignment"),
    (dict(w=FAKE + 8), _lib.WF_ERR_UNSUPPORTED, "alignment"),
])
def test_layernorm_contract_errors(lib, kw, code, msg):
    assert _ln(lib, **kw) == code
    assert msg in _lib.last_error()


def test_layernorm_empty_is_noop(lib):
    assert _ln(lib, rows=0) == _lib.WF_OK


def test_probe_gather_contract_errors(lib):
    s4 = _i64(64 * 8 * 64, 64, 8 * 64, 1)
    si = _i64(64 * 8, 8, 1)
    call = lambda **kw: lib.wf_probe_gather(  # noqa: E731
        kw.get("k", FAKE), FAKE, kw.get("dtype", 2), 1, 8, 64, kw.get("D", 64), s4, s4,
        kw.get("idx", FAKE), si, kw.get("K", 8), FAKE, kw.get("sink", 1 << 20), None)
    assert call(dtype=0) == _lib.WF_ERR_UNSUPPORTED and "16-bit" in _lib.last_error()
    assert call(D=96) == _lib.WF_ERR_INVALID_ARGUMENT
    assert call(K=6) == _lib.WF_ERR_UNSUPPORTED
    assert call(k=None) == _lib.WF_ERR_INVALID_ARGUMENT
    assert call(idx=FAKE + 4) == _lib.WF_ERR_UNSUPPORTED and "fast layout" in _lib.last_error()
    assert call(sink=16) == _lib.WF_ERR_WORKSPACE
    assert lib.wf_probe_gather_sink_bytes(1, 8, 64) == 8 * 4 * 256 * 4   # 8 pairs x 4 workgroups of 16 rows


def test_fused_pass_flags_contract(lib):
    """WF_FLAG_SINGLE_PASS on a shape the single-pass kernel does not take, and both pass
    flags at once, are reported before any kernel launch."""
    a = _lib.FusedArgs()
    a.q_search = a.k_search = a.q = a.k = a.v = a.out = a.out_idx = FAKE
    a.workspace, a.workspace_bytes = FAKE, 1 << 20
    B, H, T, D, R = 1, 2, 64, 32, 32
    a.qs_strides[:] = [T * R, R, 1]
    a.ks_strides[:] = [T * R, R, 1]
    for name in ("q_strides", "k_strides", "v_strides", "out_strides"):
        getattr(a, name)[:] = [T * H * D, D, H * D, 1]
    a.B, a.H, a.T, a.D, a.R, a.top_k = B, H, T, D, R, 16
    a.search_dtype = a.dtype = 2
    a.scale = 0.1
    a.flags = _lib.WF_FLAG_SINGLE_PASS
    assert lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), None) == _lib.WF_ERR_UNSUPPORTED
    assert "single-pass" in _lib.last_error()
    a.flags = _lib.WF_FLAG_SINGLE_PASS | _lib.WF_FLAG_SPLIT_PASS
    assert lib.wf_fused_topk_sparse_fwd(ctypes.byref(a), None) == _lib.WF_ERR_INVALID_ARGUMENT
