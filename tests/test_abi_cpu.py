"""The C-ABI library loads, exports every symbol include/holo_mi355x.h
declares, and rejects bad arguments on the host (no kernel is launched)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from holonomyawareattention_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "holo_mi355x.h")


def _declared():
    text = open(HEADER).read()
    return re.findall(r"HOLO_API\s+[\w\s\*]+?\b(holo_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_entry_points():
    names = _declared()
    assert set(names) == {n for n, _, _ in _lib.SIGNATURES}
    assert "holo_geom_scan_fwd" in names and "holo_attn_fwd" in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_exported_symbols_are_exactly_the_abi():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("holo_")}
    assert exported == set(_declared())


def test_version_and_layout_queries(lib):
    assert lib.holo_abi_version() >> 16 >= 6
    assert [lib.holo_padded_head_dim(d) for d in (1, 12, 32, 33, 48, 96)] == [32, 32, 32, 64, 64, 96]
    assert [lib.holo_padded_seq_len(t) for t in (1, 64, 65, 2048)] == [64, 64, 128, 2048]
    # chained-scan workspace: 256 bytes for the ticket counter and status word,
    # then fp32 quaternions for every chunk product and every chunk inclusive
    # prefix per (b, h, block)
    assert lib.holo_geom_scan_workspace_size(16, 2048, 16, 96) == 16 * 16 * 2 * 32 * 32 * 16 + 256
    assert lib.holo_geom_scan_workspace_size(1, 1, 1, 2) == 256
    assert lib.holo_geom_scan_workspace_size(0, 2048, 16, 96) == 0


def _scan(lib, **kw):
    args = dict(B=1, T=8, H=2, d=12, gen=0, es=0.1, io=_lib.HOLO_F32, op=_lib.HOLO_F32, gdt=_lib.HOLO_F32,
                pf=_lib.HOLO_QUAT_F32,
                mode=_lib.HOLO_MODE_CAUSAL, gq=16, gk=16, q=16, k=16, v=16, qh=16, kh=16, vh=16, P=16, hol=None, ws=16, wsb=1 << 20,
                rs=64, hs=24)
    args.update(kw)
    a = args
    return lib.holo_geom_scan_fwd(a["B"], a["T"], a["H"], a["d"], a["gen"], a["es"], a["io"], a["op"], a["gdt"],
                                  a["pf"],
                                  a["mode"], a["gq"], a["rs"], a["hs"], a["gk"], a["rs"], a["hs"],
                                  a["q"], a["rs"], a["hs"], a["k"], a["rs"], a["hs"], a["v"], a["rs"], a["hs"],
                                  a["qh"], a["kh"], a["vh"], a["P"], a["hol"], a["ws"], a["wsb"], None)


def test_scan_argument_validation(lib):
    assert _scan(lib, B=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert b"positive" in lib.holo_last_error()
    assert _scan(lib, d=200) == _lib.HOLO_ERR_UNSUPPORTED
    assert _scan(lib, io=7) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, pf=2) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, mode=2) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, io=_lib.HOLO_F32, gdt=_lib.HOLO_BF16) == _lib.HOLO_ERR_UNSUPPORTED
    assert _scan(lib, op=_lib.HOLO_F16) == _lib.HOLO_ERR_INVALID_ARG            # fp32 inputs: fp32 operands
    assert _scan(lib, io=_lib.HOLO_BF16, op=_lib.HOLO_F32) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, io=_lib.HOLO_BF16, op=9) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, k=None) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, gen=_lib.HOLO_GEN_ADDITIVE, gk=None) == _lib.HOLO_ERR_INVALID_ARG
    assert _scan(lib, gen=_lib.HOLO_GEN_DIRECT) == _lib.HOLO_ERR_INVALID_ARG      # gk given
    assert _scan(lib, hs=4) == _lib.HOLO_ERR_INVALID_ARG                          # heads overlap
    assert _scan(lib, kh=8) == _lib.HOLO_ERR_INVALID_ARG                          # misaligned
    assert _scan(lib, wsb=16) == _lib.HOLO_ERR_WORKSPACE
    assert _scan(lib, ws=None) == _lib.HOLO_ERR_WORKSPACE


def test_attention_argument_validation(lib):
    F32, BF16, F16 = _lib.HOLO_F32, _lib.HOLO_BF16, _lib.HOLO_F16

    def f(B, T, H, d, op, out, pf, sc, qh, kh, vh, P, o, rs, hs, lse):
        return lib.holo_attn_fwd(B, T, H, d, op, out, pf, sc, qh, kh, vh, P, o, rs, hs, lse, None)
    assert f(1, 0, 1, 12, F32, F32, 0, 0.3, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_BAD_SHAPE
    assert f(1, 8, 1, 120, F32, F32, 0, 0.3, 16, 16, 16, 16, 16, 120, 120, None) == _lib.HOLO_ERR_UNSUPPORTED
    assert f(1, 8, 1, 12, F32, F32, 0, 0.0, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, F32, F32, 0, 0.3, None, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 2, 12, F32, F32, 0, 0.3, 16, 16, 16, 16, 16, 12, 4, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, 5, F32, 0, 0.3, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, F32, BF16, 0, 0.3, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, F16, F16, 0, 0.3, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, F32, F32, 3, 0.3, 16, 16, 16, 16, 16, 12, 12, None) == _lib.HOLO_ERR_INVALID_ARG
    assert f(1, 8, 1, 12, F32, F32, 0, 0.3, 16, 16, 16, 16, 16, 12, 12, 8) == _lib.HOLO_ERR_INVALID_ARG   # lse misaligned


def test_projection_argument_validation(lib):
    f = lib.holo_qkvg_proj_fwd

    def call(M=512, T=256, K=128, nq=384, ng=96, xs=128, qs=384, gs=96, x=16, wq=16, w0=16, w1=16, q=16, g=16):
        return f(M, T, K, nq, ng, x, xs, wq, w0, w1, q, qs, g, gs, None)
    assert call(M=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert call(T=300) == _lib.HOLO_ERR_BAD_SHAPE                   # M not a whole number of sequences
    assert call(K=96, xs=96) == _lib.HOLO_ERR_UNSUPPORTED            # K not a multiple of 64
    assert call(nq=386, qs=392) == _lib.HOLO_ERR_UNSUPPORTED         # output width not a multiple of 4
    assert call(x=None) == _lib.HOLO_ERR_INVALID_ARG
    assert call(w0=None) == _lib.HOLO_ERR_INVALID_ARG                # generator weights needed when ng > 0
    assert call(q=8) == _lib.HOLO_ERR_INVALID_ARG                    # misaligned
    assert call(qs=388) == _lib.HOLO_ERR_INVALID_ARG                 # qkv row stride not a 16-byte multiple
    assert call(xs=120) == _lib.HOLO_ERR_INVALID_ARG                 # x row stride below K


def test_edge_gemm_argument_validation(lib):
    h = lib.holo_edge_hidden_fwd

    def hidden(M=512, T=256, K=128, nq=384, nh=512, xs=128, w1s=256, hs=512, qs=384,
               x=16, wq=16, w1=16, b1=16, q=16, hid=16):
        return h(M, T, K, nq, nh, x, xs, wq, w1, w1s, b1, q, qs, hid, hs, None)
    assert hidden(nh=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert hidden(T=300) == _lib.HOLO_ERR_BAD_SHAPE
    assert hidden(K=96, xs=96, w1s=192) == _lib.HOLO_ERR_UNSUPPORTED
    assert hidden(nh=510, hs=512) == _lib.HOLO_ERR_UNSUPPORTED        # hidden width not a multiple of 4
    assert hidden(b1=None) == _lib.HOLO_ERR_INVALID_ARG               # the bias is required
    assert hidden(wq=None) == _lib.HOLO_ERR_INVALID_ARG               # q/k/v weights needed when nq > 0
    assert hidden(hid=8) == _lib.HOLO_ERR_INVALID_ARG                 # misaligned
    assert hidden(w1s=248) == _lib.HOLO_ERR_INVALID_ARG               # W1 rows shorter than 2K
    assert hidden(hs=508) == _lib.HOLO_ERR_INVALID_ARG                # hid row stride not a 16-byte multiple
    # W1 read to the end of its last 256-row tile: 1024 * 2^20 * 2 bytes is 2 GiB
    assert hidden(K=1 << 19, xs=1 << 19, w1s=1 << 20, nq=0, nh=1000, hs=1000, M=1, T=1) == _lib.HOLO_ERR_UNSUPPORTED
    g = lib.holo_gemm_f32out_fwd

    def out(M=512, K=512, N=120, as_=512, cs=120, a=16, w=16, c=16):
        return g(M, K, N, a, as_, w, c, cs, None)
    assert out(N=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert out(K=500, as_=504) == _lib.HOLO_ERR_UNSUPPORTED
    assert out(N=126, cs=128) == _lib.HOLO_ERR_UNSUPPORTED            # width not a multiple of 4
    assert out(w=None) == _lib.HOLO_ERR_INVALID_ARG
    assert out(c=4) == _lib.HOLO_ERR_INVALID_ARG
    assert out(cs=118) == _lib.HOLO_ERR_INVALID_ARG                   # c row stride below N
    assert out(as_=508) == _lib.HOLO_ERR_INVALID_ARG                  # a row stride not a 16-byte multiple
    assert out(M=1 << 22, as_=512) == _lib.HOLO_ERR_UNSUPPORTED       # a above 2 GiB


def test_workspace_status_validation(lib):
    st = lib.holo_workspace_status
    assert st(None, 1024, 16, None) == _lib.HOLO_ERR_INVALID_ARG
    assert st(16, 1024, None, None) == _lib.HOLO_ERR_INVALID_ARG
    assert st(16, 4, 16, None) == _lib.HOLO_ERR_WORKSPACE


def _bwd(lib, **kw):
    a = dict(B=1, T=8, H=2, d=12, gen=0, es=0.1, io=_lib.HOLO_F32, gdt=_lib.HOLO_F32, sc=0.3,
             gq=16, gk=16, qh=16, kh=16, vh=16, P=16, lse=16, o=16, do=16, dq=16, dk=16, dv=16,
             dgq=16, dgk=16, ws=16, wsb=1 << 30, rs=64, hs=24, grs=64, ghs=24)
    a.update(kw)
    return lib.holo_attn_bwd(a["B"], a["T"], a["H"], a["d"], a["gen"], a["es"], a["io"], a["gdt"], a["sc"],
                             a["gq"], a["grs"], a["ghs"], a["gk"], a["grs"], a["ghs"],
                             a["qh"], a["kh"], a["vh"], a["P"], a["lse"],
                             a["o"], a["rs"], a["hs"], a["do"], a["rs"], a["hs"],
                             a["dq"], a["rs"], a["hs"], a["dk"], a["rs"], a["hs"], a["dv"], a["rs"], a["hs"],
                             a["dgq"], a["grs"], a["ghs"], a["dgk"], a["grs"], a["ghs"],
                             a["ws"], a["wsb"], None)


def test_backward_argument_validation(lib):
    # workspace: io-dtype path-frame arrays (doh, vh; fp32 also doh_t, qh_t,
    # kh_t), delta, three fp32 arrays, the chained suffix sums and the ticket
    # block, each rounded to 256 bytes
    n = 2 * 3 * 2048 * 96
    r = lambda x: (x + 255) // 256 * 256
    rest = r(2 * 3 * 2048 * 4) + 3 * r(4 * n) + r(2 * 3 * 32 * 32 * 16) + 256
    assert lib.holo_attn_bwd_workspace_size(2, 2048, 3, 96, _lib.HOLO_BF16) == 2 * r(2 * n) + rest
    assert lib.holo_attn_bwd_workspace_size(2, 2048, 3, 96, _lib.HOLO_F32) == 5 * r(4 * n) + rest
    assert lib.holo_attn_bwd_workspace_size(2, 2048, 3, 96, 9) == 0
    assert _bwd(lib, B=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert _bwd(lib, d=200) == _lib.HOLO_ERR_UNSUPPORTED
    assert _bwd(lib, gdt=_lib.HOLO_BF16) == _lib.HOLO_ERR_UNSUPPORTED     # the backward takes an fp32 generator
    assert _bwd(lib, gen=5) == _lib.HOLO_ERR_INVALID_ARG
    assert _bwd(lib, lse=None) == _lib.HOLO_ERR_INVALID_ARG
    assert _bwd(lib, gk=None) == _lib.HOLO_ERR_INVALID_ARG               # additive needs gk / dgk
    assert _bwd(lib, hs=4) == _lib.HOLO_ERR_INVALID_ARG                  # heads overlap
    assert _bwd(lib, P=8) == _lib.HOLO_ERR_INVALID_ARG                   # misaligned
    assert _bwd(lib, sc=0.0) == _lib.HOLO_ERR_INVALID_ARG
    assert _bwd(lib, wsb=1024) == _lib.HOLO_ERR_WORKSPACE
    assert _bwd(lib, ws=None) == _lib.HOLO_ERR_WORKSPACE


def test_status_codes_map_to_reference_exceptions(lib):
    _scan(lib, B=0)
    with pytest.raises(ValueError):
        _lib.check(_lib.HOLO_ERR_BAD_SHAPE, "scan")
    _scan(lib, d=200)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.HOLO_ERR_UNSUPPORTED, "scan")
    with pytest.raises(_lib.HoloError):
        _lib.check(_lib.HOLO_ERR_WORKSPACE, "scan")
    _lib.check(_lib.HOLO_OK, "scan")


def _dgeom(lib, **kw):
    a = dict(B=1, H=2, d=12, t=3, cap=64, gen=0, es=0.1, io=_lib.HOLO_F32, gdt=_lib.HOLO_F32,
             gq=16, gk=16, q=16, k=16, v=16, P=16, qh=16, kc=16, vc=16, bs=48, hs=24)
    a.update(kw)
    return lib.holo_decode_geom_fwd(a["B"], a["H"], a["d"], a["t"], a["cap"], a["gen"], a["es"], a["io"], a["gdt"],
                                    a["gq"], a["bs"], a["hs"], a["gk"], a["bs"], a["hs"],
                                    a["q"], a["bs"], a["hs"], a["k"], a["bs"], a["hs"], a["v"], a["bs"], a["hs"],
                                    a["P"], a["qh"], a["kc"], a["vc"], None)


def test_decode_argument_validation(lib):
    assert _dgeom(lib, t=64) == _lib.HOLO_ERR_BAD_SHAPE                 # t >= capacity
    assert _dgeom(lib, cap=100) == _lib.HOLO_ERR_BAD_SHAPE              # capacity not a multiple of 64
    assert _dgeom(lib, gk=None) == _lib.HOLO_ERR_INVALID_ARG            # additive needs gk when t > 0
    assert _dgeom(lib, gen=_lib.HOLO_GEN_DIRECT) == _lib.HOLO_ERR_INVALID_ARG   # direct takes no gk
    assert _dgeom(lib, kc=8) == _lib.HOLO_ERR_INVALID_ARG               # misaligned cache
    assert _dgeom(lib, d=200) == _lib.HOLO_ERR_UNSUPPORTED
    f = lib.holo_decode_attn_fwd
    need = lib.holo_decode_attn_workspace_size(1, 2, 12, 300)
    assert need == 1 * 2 * 2 * (32 + 2) * 4                             # two 256-key segments at t = 300
    assert f(1, 2, 12, 300, 320, 0, 0.3, 16, 16, 16, 16, 16, 24, 12, 16, 16, None) == _lib.HOLO_ERR_WORKSPACE
    assert f(1, 2, 12, 400, 320, 0, 0.3, 16, 16, 16, 16, 16, 24, 12, 16, need, None) == _lib.HOLO_ERR_BAD_SHAPE
    assert f(1, 2, 12, 3, 64, 0, 0.3, 16, 16, 16, 16, 16, 24, 4, 16, need, None) == _lib.HOLO_ERR_INVALID_ARG


def _addln(lib, **kw):
    a = dict(n=4, d=96, dt=_lib.HOLO_F32, eps=1e-5, x=16, xs=96, dl=16, ds=96, w=16, b=16, h=16, hs=96,
             y=16, ys=96)
    a.update(kw)
    return lib.holo_add_layernorm_fwd(a["n"], a["d"], a["dt"], a["eps"], a["x"], a["xs"], a["dl"], a["ds"],
                                      a["w"], a["b"], a["h"], a["hs"], a["y"], a["ys"], None)


def test_add_layernorm_argument_validation(lib):
    assert _addln(lib, n=0) == _lib.HOLO_OK                               # no rows: nothing launched
    assert _addln(lib, n=-1) == _lib.HOLO_ERR_BAD_SHAPE
    assert _addln(lib, d=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert _addln(lib, dt=7) == _lib.HOLO_ERR_INVALID_ARG
    assert _addln(lib, d=98) == _lib.HOLO_ERR_UNSUPPORTED                 # not a 16-byte multiple (fp32)
    assert _addln(lib, d=100, dt=_lib.HOLO_BF16, xs=104, ds=104, hs=104, ys=104) == _lib.HOLO_ERR_UNSUPPORTED
    assert _addln(lib, d=4100, xs=4100, ds=4100, hs=4100, ys=4100) == _lib.HOLO_ERR_UNSUPPORTED   # > 4096 fp32
    assert _addln(lib, eps=0.0) == _lib.HOLO_ERR_INVALID_ARG
    assert _addln(lib, w=None) == _lib.HOLO_ERR_INVALID_ARG
    assert _addln(lib, xs=90) == _lib.HOLO_ERR_INVALID_ARG                # stride below d
    assert _addln(lib, ys=98) == _lib.HOLO_ERR_INVALID_ARG                # stride not a 16-byte multiple
    assert _addln(lib, h=8) == _lib.HOLO_ERR_INVALID_ARG                  # misaligned


def _masked(lib, **kw):
    a = dict(B=1, T=8, H=2, d=12, dt=_lib.HOLO_F32, pf=_lib.HOLO_QUAT_F32, mode=_lib.HOLO_MODE_CAUSAL, sc=0.3,
             qh=16, kh=16, vh=16, P=16, hol=16, mask=16, mrs=8, o=16, rs=24, hs=12, ws=16, wsb=1 << 20)
    a.update(kw)
    return lib.holo_attn_masked_fwd(a["B"], a["T"], a["H"], a["d"], a["dt"], a["pf"], a["mode"], a["sc"],
                                    a["qh"], a["kh"], a["vh"], a["P"], a["hol"], a["mask"], a["mrs"],
                                    a["o"], a["rs"], a["hs"], a["ws"], a["wsb"], None)


def test_masked_attention_argument_validation(lib):
    ws = lib.holo_attn_masked_workspace_size
    # with a mask: Tp * Tp/64 mask words and the ceil(T/128) x Tp/64 map of open tiles
    assert ws(2, 100, 3, 48, _lib.HOLO_BF16, _lib.HOLO_MODE_CAUSAL, 1) == 128 * 2 * 8 + 1 * 2
    assert ws(2, 300, 3, 48, _lib.HOLO_F32, _lib.HOLO_MODE_INERT, 1) == 320 * 5 * 8 + 3 * 5
    assert ws(2, 100, 3, 48, _lib.HOLO_BF16, _lib.HOLO_MODE_CAUSAL, 0) == 0
    assert ws(2, 100, 3, 48, 9, _lib.HOLO_MODE_INERT, 0) == 0
    assert _masked(lib, T=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert _masked(lib, d=120) == _lib.HOLO_ERR_UNSUPPORTED
    assert _masked(lib, mode=2) == _lib.HOLO_ERR_INVALID_ARG
    assert _masked(lib, dt=3) == _lib.HOLO_ERR_INVALID_ARG
    assert _masked(lib, dt=_lib.HOLO_F16) == _lib.HOLO_ERR_INVALID_ARG   # the exact path takes bf16 / fp32
    assert _masked(lib, pf=5) == _lib.HOLO_ERR_INVALID_ARG
    assert _masked(lib, hol=None) == _lib.HOLO_ERR_INVALID_ARG            # causal mode needs the holonomy
    assert _masked(lib, mrs=7) == _lib.HOLO_ERR_INVALID_ARG               # mask rows shorter than T
    assert _masked(lib, hs=4) == _lib.HOLO_ERR_INVALID_ARG                # output heads overlap
    assert _masked(lib, kh=8) == _lib.HOLO_ERR_INVALID_ARG                # misaligned
    assert _masked(lib, sc=0.0) == _lib.HOLO_ERR_INVALID_ARG
    assert _masked(lib, wsb=64) == _lib.HOLO_ERR_WORKSPACE
    assert _masked(lib, ws=None) == _lib.HOLO_ERR_WORKSPACE
    assert _masked(lib, mask=None, ws=None, wsb=0, T=0) == _lib.HOLO_ERR_BAD_SHAPE   # no mask: no workspace


def _mbwd(lib, **kw):
    a = dict(B=1, T=8, H=2, d=12, gen=0, es=0.1, io=_lib.HOLO_F32, gdt=_lib.HOLO_F32, mode=_lib.HOLO_MODE_CAUSAL,
             sc=0.3, gq=16, gk=16, qh=16, kh=16, vh=16, P=16, hol=16, lse=16, mask=16, mrs=8, o=16, do=16, dq=16,
             dk=16, dv=16, dgq=16, dgk=16, ws=16, wsb=1 << 30, rs=64, hs=24, grs=64, ghs=24)
    a.update(kw)
    return lib.holo_attn_masked_bwd(a["B"], a["T"], a["H"], a["d"], a["gen"], a["es"], a["io"], a["gdt"], a["mode"],
                                    a["sc"], a["gq"], a["grs"], a["ghs"], a["gk"], a["grs"], a["ghs"],
                                    a["qh"], a["kh"], a["vh"], a["P"], a["hol"], a["lse"], a["mask"], a["mrs"],
                                    a["o"], a["rs"], a["hs"], a["do"], a["rs"], a["hs"],
                                    a["dq"], a["rs"], a["hs"], a["dk"], a["rs"], a["hs"], a["dv"], a["rs"], a["hs"],
                                    a["dgq"], a["grs"], a["ghs"], a["dgk"], a["grs"], a["ghs"],
                                    a["ws"], a["wsb"], None)


def test_exact_path_training_argument_validation(lib):
    ws = lib.holo_attn_masked_bwd_workspace_size
    base = lib.holo_attn_bwd_workspace_size(2, 300, 3, 48, _lib.HOLO_BF16)
    r = lambda x: (x + 255) // 256 * 256
    n = 2 * 3 * 320 * 64
    # inert mode, no mask: the tril backward's workspace; a mask adds its bits
    # and tile map; causal mode adds qw, dow (bf16), dqw, dkw, dvw and the
    # holonomy's cross sums
    assert ws(2, 300, 3, 48, _lib.HOLO_BF16, _lib.HOLO_MODE_INERT, 0) == base
    assert ws(2, 300, 3, 48, _lib.HOLO_BF16, _lib.HOLO_MODE_INERT, 1) == base + r(320 * 5 * 8) + r(3 * 5)
    assert ws(2, 300, 3, 48, _lib.HOLO_BF16, _lib.HOLO_MODE_CAUSAL, 0) == \
        base + 2 * r(2 * n) + 3 * r(4 * n) + r(2 * 3 * 16 * 16)
    assert ws(2, 300, 3, 48, _lib.HOLO_F32, _lib.HOLO_MODE_CAUSAL, 0) == \
        lib.holo_attn_bwd_workspace_size(2, 300, 3, 48, _lib.HOLO_F32) + 4 * r(4 * n) + 3 * r(4 * n) + r(2 * 3 * 16 * 16)
    assert ws(2, 300, 3, 48, _lib.HOLO_BF16, 7, 0) == 0
    assert _mbwd(lib, B=0) == _lib.HOLO_ERR_BAD_SHAPE
    assert _mbwd(lib, mode=3) == _lib.HOLO_ERR_INVALID_ARG
    assert _mbwd(lib, hol=None) == _lib.HOLO_ERR_INVALID_ARG             # causal mode needs the holonomy
    assert _mbwd(lib, hol=8) == _lib.HOLO_ERR_INVALID_ARG                # misaligned
    assert _mbwd(lib, mrs=7) == _lib.HOLO_ERR_INVALID_ARG                # mask rows shorter than T
    assert _mbwd(lib, lse=None) == _lib.HOLO_ERR_INVALID_ARG
    assert _mbwd(lib, gdt=_lib.HOLO_BF16) == _lib.HOLO_ERR_UNSUPPORTED
    assert _mbwd(lib, wsb=1024) == _lib.HOLO_ERR_WORKSPACE
    t = lib.holo_attn_masked_train_fwd
    args = lambda lse: (1, 8, 2, 12, _lib.HOLO_F32, _lib.HOLO_MODE_CAUSAL, 0.3, 16, 16, 16, 16, 16, 16, 8,
                        16, 24, 12, lse, 16, 1 << 20, None)
    assert t(*args(None)) == _lib.HOLO_ERR_INVALID_ARG                    # the LSE is the point of this call
    assert t(*args(8)) == _lib.HOLO_ERR_INVALID_ARG                       # misaligned LSE


def test_dropout_argument_validation(lib):
    """The dropout entry points refuse a probability outside [0, 1) (NaN
    included), a null LSE or keep buffer and the exact path's other invalid
    arguments before any launch."""
    f = lib.holo_attn_masked_dropout_fwd
    fargs = lambda p, lse=16, B=1: (B, 8, 2, 12, _lib.HOLO_F32, _lib.HOLO_MODE_CAUSAL, 0.3, p, 2 ** 64 - 1, 7,
                                    16, 16, 16, 16, 16, 16, 8, 16, 24, 12, lse, 16, 1 << 20, None)
    for p in (-0.1, 1.0, 1.5, float("nan"), float("inf")):
        assert f(*fargs(p)) == _lib.HOLO_ERR_INVALID_ARG, p
        assert "dropout probability" in lib.holo_last_error().decode()
    assert f(*fargs(0.1, lse=None)) == _lib.HOLO_ERR_INVALID_ARG
    assert f(*fargs(0.1, lse=8)) == _lib.HOLO_ERR_INVALID_ARG            # misaligned LSE
    assert f(*fargs(0.1, B=0)) == _lib.HOLO_ERR_BAD_SHAPE
    b = lib.holo_attn_masked_dropout_bwd
    bargs = lambda p, **kw: (1, 8, 2, 12, 0, 0.1, _lib.HOLO_F32, _lib.HOLO_F32, kw.get("mode", _lib.HOLO_MODE_CAUSAL),
                             0.3, p, 5, 0, 16, 64, 24, 16, 64, 24, 16, 16, 16, 16, kw.get("hol", 16), 16, 16, 8,
                             16, 64, 24, 16, 64, 24, 16, 64, 24, 16, 64, 24, 16, 64, 24, 16, 64, 24, 16, 64, 24,
                             16, 1 << 30, None)
    assert b(*bargs(1.0)) == _lib.HOLO_ERR_INVALID_ARG
    assert b(*bargs(-1e-7)) == _lib.HOLO_ERR_INVALID_ARG
    assert b(*bargs(0.2, mode=3)) == _lib.HOLO_ERR_INVALID_ARG
    assert b(*bargs(0.2, hol=None)) == _lib.HOLO_ERR_INVALID_ARG
    k = lib.holo_dropout_keep_mask
    assert k(1, 8, 2, 0.1, 1, 0, None, None) == _lib.HOLO_ERR_INVALID_ARG
    assert k(1, 8, 2, 1.0, 1, 0, 16, None) == _lib.HOLO_ERR_INVALID_ARG
    assert k(0, 8, 2, 0.1, 1, 0, 16, None) == _lib.HOLO_ERR_BAD_SHAPE
    assert k(1, 0, 2, 0.1, 1, 0, 16, None) == _lib.HOLO_ERR_BAD_SHAPE
