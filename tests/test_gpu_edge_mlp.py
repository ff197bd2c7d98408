"""The interaction generator on the hand-written GEMM: holo_edge_hidden_fwd
(q/k/v and the edge MLP's first layer on the token rows t and t+1, bias and
exact GELU in the epilogue; core/attention_fast_chunked.py:56-60,69-76) and
holo_gemm_f32out_fwd (the second layer on the same GEMM, fp32 output),
through kernels.edge_hidden and kernels.edge_out, against float64 products
of the same bf16 inputs; then the module's bf16 interaction path with
fused_interaction on against the oracle.

Bounds (written in the test): the bf16 x bf16 products are exact in fp32 and
the K-term sums (bias included) are accumulated in fp32, so any order is
within K * 2^-24 * sum_c |x_c w_c| of the exact sum; as the reference's bf16
Linear does, the pre-activation is rounded to bf16 (unit roundoff 2^-8) before
GELU, whose slope is below 1.13, so the pre-activation errors reach the hidden
value at most 1.2 times; GELU in fp32 with erf from Abramowitz & Stegun 7.1.26
(|error| < 1.5e-7, so 0.5 |v| 1.5e-7 on GELU) adds at most 2^-22 (|pre| + |h|);
the hidden values and q/k/v are rounded once more to bf16. The second layer's
4D-term sums are stored in fp32. Per-head o: max-abs <= 2e-3 against the
oracle fed the GPU's own q, k, v and generator output (the bar of the
additive path).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy.special import erf

from holonomyawareattention_amd import kernels
from oracle import holo_ref as R
from tests._util import layer, make_module, run_module

pytestmark = [
    pytest.mark.gpu,
    # The fused interaction generator has been executed only on the CPU
    # emulation of the kernels (tests/test_emu_kernels.py, at these shapes
    # and at config 2's): GPU use for the repository was closed before it
    # could run on a GPU. Two earlier implementations of the path ended their
    # first GPU run in a fault whose cause was not found. The module keeps it
    # off (fused_interaction = False) and these tests stay skipped until they
    # can run on a GPU.
    pytest.mark.skip(reason="fused interaction generator not yet run on a GPU (executed on the CPU emulation only)"),
]
DEV = torch.device("cuda:0")
BAR = 2e-3


def _gelu(v):
    return 0.5 * v * (1.0 + erf(v / math.sqrt(2.0)))


def _check_gemms(B, T, D, H, seed, rows=None):
    x, W = layer(seed, B, T, D, H, "interaction", dtype=torch.bfloat16)
    xt = torch.as_tensor(x).to(DEV, torch.bfloat16)
    dv = lambda k: torch.as_tensor(W[k]).to(DEV, torch.bfloat16).contiguous()
    wq, w1, b1, w2 = dv("qkv.weight"), dv("edge_mlp.0.weight"), dv("edge_mlp.0.bias"), dv("edge_mlp.2.weight")
    qkv, hid = kernels.edge_hidden(xt, wq, w1, b1)
    g = kernels.edge_out(hid, w2)
    _, hid_only = kernels.edge_hidden(xt, None, w1, b1)            # the hidden layer alone (no q/k/v tiles)
    torch.cuda.synchronize()
    assert torch.equal(hid, hid_only)
    r = np.arange(B * T) if rows is None else np.asarray(rows)
    ri = torch.as_tensor(r, device=DEV)
    xs = x.reshape(B * T, D)[r]
    xn = np.roll(x, -1, axis=1).reshape(B * T, D)[r]                 # x_{(t+1) mod T} of the same sequence
    W1 = np.asarray(W["edge_mlp.0.weight"])
    W1a, W1b, bias = W1[:, :D], W1[:, D:], np.asarray(W["edge_mlp.0.bias"])
    pre = xs @ W1a.T + xn @ W1b.T + bias
    mag = np.abs(xs) @ np.abs(W1a).T + np.abs(xn) @ np.abs(W1b).T + np.abs(bias)
    ref_h = _gelu(pre)
    got_h = hid.reshape(B * T, -1)[ri].double().cpu().numpy()
    bh = (2.0 ** -8 * np.abs(ref_h) + 1.2 * 2.0 ** -8 * np.abs(pre) + 1.2 * (2 * D + 1) * 2.0 ** -24 * mag
          + 2.0 ** -22 * (np.abs(pre) + np.abs(ref_h)))
    eh = np.abs(got_h - ref_h)
    Wq = np.asarray(W["qkv.weight"])
    ref_q, mag_q = xs @ Wq.T, np.abs(xs) @ np.abs(Wq).T
    got_q = qkv.reshape(B * T, -1)[ri].double().cpu().numpy()
    bq = 2.0 ** -8 * np.abs(ref_q) + (1 + 2.0 ** -8) * D * 2.0 ** -24 * mag_q
    eq = np.abs(got_q - ref_q)
    W2 = np.asarray(W["edge_mlp.2.weight"])
    ref_g, mag_g = got_h @ W2.T, np.abs(got_h) @ np.abs(W2).T    # the second layer on the GPU's own hidden values
    got_g = g.reshape(B * T, -1)[ri].double().cpu().numpy()
    bg = 4 * D * 2.0 ** -24 * mag_g
    eg = np.abs(got_g - ref_g)
    print(f"B={B} T={T} D={D} H={H}: hidden max err {eh.max():.3e} (err/bound {(eh / bh).max():.3f}), "
          f"qkv {eq.max():.3e} ({(eq / bq).max():.3f}), g {eg.max():.3e} ({(eg / bg).max():.3f})")
    assert np.all(eh <= bh) and np.all(eq <= bq) and np.all(eg <= bg)


def test_edge_mlp_cfg2_rows():
    """Config 2's layer in interaction mode (M = 32768, D = 1536: hidden width
    6144 over 2D = 3072, second layer 6144 -> 1536): batch row 0 whole and
    the last two tokens of every other sequence (the wrap to token 0)."""
    B, T, D, H = 16, 2048, 1536, 16
    rows = np.concatenate([np.arange(T)] + [[b * T + T - 2, b * T + T - 1] for b in range(1, B)])
    _check_gemms(B, T, D, H, 61, rows)


@pytest.mark.parametrize("B,T,D,H", [(3, 100, 128, 4), (5, 1, 128, 4), (2, 257, 192, 4)])
def test_edge_mlp_ragged_shapes(B, T, D, H):
    """M and the widths not multiples of the 256 x 256 tile; T = 1 (every
    token's successor is itself)."""
    _check_gemms(B, T, D, H, 62)


def test_module_interaction_per_head_output_2e3():
    """The module's bf16 interaction path as it runs (fused GEMMs, fp16
    attention operands, int16 quaternions), per-head o in fp32 against the
    oracle fed the GPU's own q, k, v and generator output g + b2: every (b, h)
    at the first 256 positions and batch row 1 at every position, config 2's
    layer at B = 2; max-abs <= 2e-3."""
    B, T, D, H, es = 2, 2048, 1536, 16, 0.05
    x, W = layer(63, B, T, D, H, "interaction", dtype=torch.bfloat16)
    m = make_module(W, D, H, es, "interaction", torch.bfloat16, DEV)
    m.fused_interaction = True
    xt = torch.as_tensor(x).to(DEV, torch.bfloat16)
    assert m._fused_interaction_ok(xt)
    with torch.no_grad():
        q, k, v, gq, gk = m._link_inputs(xt, fused=True)
        qh, kh, vh_t, P, _ = kernels.geom_scan(q, k, v, gq, gk, es, p_format="snorm16", op_dtype=torch.float16)
        o = kernels.attention(qh, kh, vh_t, P, m.d, m.scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    f64 = lambda t: t.detach().double().cpu().numpy().transpose(0, 2, 1, 3)
    a = es * (f64(gq) + f64(gk))                                    # gk: the bias, a per-head constant
    Pq, _ = R.geometry_blocks(a)
    og = f64(o)
    qq, kk, vv = (R.apply_blocks_T(Pq, f64(u)) for u in (q, k, v))
    rows = np.arange(256)
    ref = R.apply_blocks(Pq[:, :, rows], R.attention_rows64(qq, kk, vv, m.scale, rows))
    worst = np.abs(og[:, :, rows] - ref).max()
    ref1 = R.apply_blocks(Pq[1:2], R.attention_rows64(qq[1:2], kk[1:2], vv[1:2], m.scale, np.arange(T)))
    worst = max(worst, np.abs(og[1:2] - ref1).max())
    print(f"interaction per-head o: max-abs {worst:.3e}")
    assert worst <= BAR, worst


@pytest.mark.parametrize("B,T,D,H", [(2, 300, 128, 4), (1, 129, 192, 4)])
def test_module_interaction_against_oracle(B, T, D, H):
    """End to end in bf16 at shapes that take the fused path: y against the
    float64 oracle (the reference's algorithm on the block model) on the same
    bf16-rounded inputs and weights, relative Frobenius <= 1e-2 (y is stored in
    bf16; the bar of the other bf16 end-to-end checks)."""
    es = 0.5
    x, W = layer(64, B, T, D, H, "interaction", dtype=torch.bfloat16)
    m = make_module(W, D, H, es, "interaction", torch.bfloat16, DEV)
    m.fused_interaction = True
    assert m._fused_interaction_ok(torch.as_tensor(x).to(DEV, torch.bfloat16))
    y, _ = run_module(m, x, DEV, torch.bfloat16)
    ref = R.forward_blocks(x, W, H, es, "interaction")
    got = y.double().cpu().numpy()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    print(f"B={B} T={T} D={D} H={H}: relative Frobenius {rel:.3e}, max-abs {np.abs(got - ref).max():.3e}")
    assert rel <= 1e-2
