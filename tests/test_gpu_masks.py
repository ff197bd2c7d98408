"""The exact-path kernels (holo_attn_masked_fwd: any mask, causal mode with the
wrap branch through the holonomy, inert mode) against the float64 oracle
(oracle.holo_ref.forward_exact_blocks, pinned in tests/test_oracle_masks.py
against the arc-walk definition), through the drop-in module.

Tolerances (written in each test): fp32 max-abs <= 2e-5 against the oracle on
fp32-rounded inputs: the causal-path bar of 1e-5 plus the holonomy, which the
wrap branch carries and which composes all T links in fp32 (one more rounding
per link than any P_t; measured 1.2e-5 at T = 130 with edge_scale 0.9); bf16
max-abs <= 2.5e-2 and relative Frobenius <= 1e-2 against the oracle on the
bf16-rounded inputs (the bf16 bar without its absolute RMS term: a sparse mask
such as the ring mask averages three values per row, so the output keeps the
magnitude of one value and with it the absolute size of each bf16 rounding:
RMS 2.7e-3 at max-abs 1.5e-2 measured for the ring mask in causal mode). Rows
whose mask allows no key must be NaN exactly where the oracle's are (the
reference's torch.softmax over -inf only).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import kernels
from oracle import holo_ref as R
from tests._util import tril, layer, make_module

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _mask(kind, T, seed=0):
    if kind == "none":
        return None
    if kind == "ring":
        return R.ring_mask(T)
    if kind == "tril":
        return np.tril(np.ones((T, T), dtype=bool))
    m = np.random.default_rng(seed).random((T, T)) < 0.3
    m[np.arange(T), np.arange(T)] = True
    if kind == "empty_row":
        m[T // 2] = False
        m[0] = False
    return m


def _run(x, W, D, H, es, lm, dtype, mode, mask, return_geometry=False):
    m = make_module(W, D, H, es, lm, dtype, DEV)
    m.mode = mode
    xt = torch.as_tensor(x).to(device=DEV, dtype=dtype)
    mt = None if mask is None else torch.as_tensor(mask, device=DEV)
    with torch.no_grad():
        y, g = m(xt, attn_mask=mt, return_geometry=return_geometry)
    torch.cuda.synchronize()
    return y.double().cpu().numpy(), g


def _check(y, ref, dtype):
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan_ref)
    yf, rf = y[~nan_ref], ref[~nan_ref]
    err = np.abs(yf - rf)
    print(f"max-abs {err.max():.3e}")
    if dtype == torch.float32:
        assert err.max() <= 2e-5, err.max()
    else:
        rel = np.linalg.norm(yf - rf) / np.linalg.norm(rf)
        print(f"rms {np.sqrt((err ** 2).mean()):.3e} rel-F {rel:.3e}")
        assert err.max() <= 2.5e-2, err.max()
        assert rel <= 1e-2, rel


@pytest.mark.parametrize("mode", ["causal", "inert"])
@pytest.mark.parametrize("mask_kind", ["none", "ring", "random", "tril", "empty_row"])
@pytest.mark.parametrize("dtype,B,T,D,H", [(torch.float32, 2, 130, 96, 2), (torch.bfloat16, 1, 200, 192, 2),
                                           (torch.float32, 2, 70, 64, 4)])
def test_exact_path_matches_oracle(mode, mask_kind, dtype, B, T, D, H):
    if mode == "causal" and mask_kind == "tril":
        pytest.skip("causal + tril runs the causal kernels (tests/test_gpu_parity.py)")
    print(f"exact path {mode} {mask_kind} {dtype} B={B} T={T} D={D} H={H}", flush=True)
    x, W = layer(60 + T, B, T, D, H, dtype=dtype)
    mask = _mask(mask_kind, T, seed=T)
    es = 0.9
    y, _ = _run(x, W, D, H, es, "additive", dtype, mode, mask)
    with np.errstate(invalid="ignore"):
        ref = R.forward_exact_blocks(x, W, H, es, mask=mask, mode=mode)
    _check(y, ref, dtype)


@pytest.mark.parametrize("mode", ["causal", "inert"])
def test_exact_path_interaction_generator(mode):
    B, T, D, H = 2, 96, 48, 2
    x, W = layer(70, B, T, D, H, "interaction", dtype=torch.float32)
    mask = R.ring_mask(T)
    y, _ = _run(x, W, D, H, 0.7, "interaction", torch.float32, mode, mask)
    ref = R.forward_exact_blocks(x, W, H, 0.7, "interaction", mask=mask, mode=mode)
    _check(y, ref, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_exact_path_geometry_output(dtype):
    """return_geometry on the exact path (fp32 rotations between the kernels,
    also on the bf16 path): dense P and Hol equal the oracle's, within 1e-5
    (fp32) or one bf16 rounding of entries of magnitude <= 1 (4e-3)."""
    B, T, D, H = 1, 40, 48, 2
    x, W = layer(71, B, T, D, H, dtype=dtype)
    y, g = _run(x, W, D, H, 0.9, "additive", dtype, "causal", None, return_geometry=True)
    ref, parts = R.forward_exact_blocks(x, W, H, 0.9, mask=None, mode="causal", return_parts=True)
    _check(y, ref, dtype)
    d = D // H
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    assert np.abs(g["C"].double().cpu().numpy() - R.blocks_to_dense(parts["P"], d)).max() <= tol
    assert np.abs(g["H"].double().cpu().numpy() - R.blocks_to_dense(parts["Hol"], d)).max() <= tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_kernel_under_tril_equals_causal_kernel(dtype):
    """The exact-path kernel given the tril mask in causal mode computes what
    the causal kernel computes (the wrap branch fully masked): fp32 within
    2e-6, bf16 within 2^-7 relative plus 1e-3 (one bf16 rounding apart)."""
    B, T, H, d = 2, 300, 3, 96
    g = torch.Generator(device="cpu").manual_seed(5)
    q, k, v = (torch.randn(B, T, H, d, generator=g).to(DEV, dtype) for _ in range(3))
    gq, gk = ((0.3 * torch.randn(B, T, H, d, generator=g)).to(DEV) for _ in range(2))
    qh, kh, vh_t, P, hol = kernels.geom_scan(q, k, v, gq, gk, 1.0, want_hol=True, p_format="f32")
    o_fast = kernels.attention(qh, kh, vh_t, P, d, d ** -0.5)
    tril = torch.ones(T, T, dtype=torch.bool, device=DEV).tril()
    o_mask = kernels.attention_masked(qh, kh, vh_t, P, hol, d, d ** -0.5, mode="causal", mask=tril)
    torch.cuda.synchronize()
    a, b = o_mask.double(), o_fast.double()
    if dtype == torch.float32:
        assert (a - b).abs().max().item() <= 2e-6
    else:
        assert bool(((a - b).abs() <= 2.0 ** -7 * b.abs() + 1e-3).all())


def test_modes_agree_on_the_flat_connection():
    """edge_scale = 0: every transport is the identity, so causal and inert
    mode are the same masked softmax attention."""
    B, T, D, H = 2, 77, 96, 2
    x, W = layer(72, B, T, D, H, dtype=torch.float32)
    mask = _mask("random", T, seed=3)
    yc, _ = _run(x, W, D, H, 0.0, "additive", torch.float32, "causal", mask)
    yi, _ = _run(x, W, D, H, 0.0, "additive", torch.float32, "inert", mask)
    assert np.abs(yc - yi).max() <= 2e-6


def test_exact_path_under_autograd_forward_only():
    """Under autograd (x requiring grad, or only the parameters, as in an eval()
    model outside torch.no_grad()) the exact path and the geometry output run
    their forward, bit-identical to the forward with gradients off; only the
    backward raises NotImplementedError (no gfx950 backward for them)."""
    x, W = layer(73, 1, 16, 24, 2, dtype=torch.float32)
    m = make_module(W, 24, 2, 0.5, "additive", torch.float32, DEV)
    xt = torch.as_tensor(x).to(DEV, torch.float32)
    mask = tril(16, DEV)
    with torch.no_grad():
        y0, _ = m(xt, attn_mask=None)
        yg0, g0 = m(xt, attn_mask=mask, return_geometry=True)
    xg = xt.clone().requires_grad_(True)
    y1, _ = m(xg, attn_mask=None)                       # x and the parameters require grad
    assert y1.requires_grad and torch.equal(y1.detach(), y0)
    with pytest.raises(NotImplementedError, match="attention mask other than tril"):
        y1.sum().backward()
    y2, _ = m.eval()(xt, attn_mask=None)                # only the parameters require grad
    assert y2.requires_grad and torch.equal(y2.detach(), y0)
    yg1, g1 = m(xg, attn_mask=mask, return_geometry=True)
    assert torch.equal(yg1.detach(), yg0)
    assert torch.equal(g1["C"].detach(), g0["C"]) and torch.equal(g1["H"].detach(), g0["H"])
    with pytest.raises(NotImplementedError, match="geometry output"):
        g1["C"].sum().backward()
    m.mode = "inert"
    y3, _ = m(xg, attn_mask=mask)
    with pytest.raises(NotImplementedError, match="inert mode"):
        y3.sum().backward()
