"""Incremental decode on the GPU against the fp64 oracle and the
full-sequence forward.

Row t of the causal forward depends on tokens 0..t only (the edge t-1 -> t
uses x_{t-1} and x_t; the closing edge only enters the holonomy), so
prefill(x[:, :T0]) followed by decode_step on tokens T0..T-1 must reproduce
the oracle's forward (oracle.holo_ref.forward_blocks on the same rounded
inputs) at rows T0..T-1, and the GPU's own full forward there.
Tolerances (written in each test): fp32 2e-5 max-abs (P_t composed step by
step instead of in chunks, attention summed per 256-key segment); bf16
against the oracle the y-level bound of the other bf16 tests (2.5e-2 *
max(1, max|y|/4)), against the GPU forward 2e-2 (the decode attention keeps
the softmax weights in fp32 where the full-sequence kernel rounds them to
16 bits for its PV MFMA).
"""
from __future__ import annotations

import pytest
import torch

import numpy as np

from holonomyawareattention_amd import kernels
from oracle import holo_ref as R
from tests._util import layer, make_module, run_module

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _tol(dtype):
    return 2e-5 if dtype == torch.float32 else 2e-2


def _oracle_tol(dtype, y_ref):
    return 2e-5 if dtype == torch.float32 else 2.5e-2 * max(1.0, np.abs(y_ref).max() / 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("lm", ["additive", "interaction"])
def test_decode_matches_full_forward(dtype, lm):
    B, T, D, H, es, T0 = 2, 100, 96, 2, 0.7, 37          # decoding crosses the 64-key tile boundary
    x, W = layer(40, B, T, D, H, lm, dtype=dtype)
    m = make_module(W, D, H, es, lm, dtype, DEV)
    y_full, _ = run_module(m, x, DEV, dtype)
    y_ref = R.forward_blocks(x, W, H, es, lm)
    xt = torch.as_tensor(x).to(DEV, dtype)
    y0, st = m.prefill(xt[:, :T0], capacity=T)
    assert (y0.float() - y_full[:, :T0].float()).abs().max().item() <= _tol(dtype)
    worst, worst_ref = 0.0, 0.0
    for t in range(T0, T):
        yt = m.decode_step(xt[:, t:t + 1], st)
        worst = max(worst, (yt[:, 0].float() - y_full[:, t].float()).abs().max().item())
        worst_ref = max(worst_ref, np.abs(yt[:, 0].double().cpu().numpy() - y_ref[:, t]).max())
    torch.cuda.synchronize()
    assert st.t == T
    assert worst <= _tol(dtype), worst
    assert worst_ref <= _oracle_tol(dtype, y_ref[:, T0:]), worst_ref


def test_decode_cache_matches_scan():
    """The rows decode appends to the caches are the scan's transported keys
    and values of the full sequence (fp32), and the running P is P_{T-1}."""
    B, T, D, H, es, T0 = 2, 140, 144, 3, 0.9, 70       # d = 48, 16 blocks
    x, W = layer(41, B, T, D, H, "additive", dtype=torch.float32)
    m = make_module(W, D, H, es, "additive", torch.float32, DEV)
    xt = torch.as_tensor(x).to(DEV, torch.float32)
    _, st = m.prefill(xt[:, :T0], capacity=T)
    for t in range(T0, T):
        m.decode_step(xt[:, t:t + 1], st)
    with torch.no_grad():
        q, k, v, gq, gk = m._link_inputs(xt)
        qh, kh, vh_t, P, _ = kernels.geom_scan(q, k, v, gq, gk, es)
    torch.cuda.synchronize()
    # |kh|, |vh| reach ~3: 5e-5 is ~1e-5 relative (70 steps of fp32 composition
    # step by step against the scan's chunked order); P entries are <= 1
    dk = (st.kh[:, :, :T] - kh[:, :, :T]).abs().max().item()
    dv = (st.vh[:, :, :vh_t.shape[2]] - vh_t).abs().max().item()
    dp = (st.P - P[:, :, T - 1]).abs().max().item()
    assert dk <= 5e-5 and dv <= 5e-5 and dp <= 1e-5, (dk, dv, dp)


def test_decode_many_segments_bf16():
    """Keys spread over several 256-key segments of the split attention."""
    B, T, D, H, es, T0 = 1, 800, 96, 2, 0.3, 790
    x, W = layer(42, B, T, D, H, "additive", dtype=torch.bfloat16)
    m = make_module(W, D, H, es, "additive", torch.bfloat16, DEV)
    y_full, _ = run_module(m, x, DEV, torch.bfloat16)
    y_ref = R.forward_blocks(x, W, H, es, "additive")
    xt = torch.as_tensor(x).to(DEV, torch.bfloat16)
    _, st = m.prefill(xt[:, :T0])
    worst, worst_ref = 0.0, 0.0
    for t in range(T0, T):
        yt = m.decode_step(xt[:, t:t + 1], st)
        worst = max(worst, (yt[:, 0].float() - y_full[:, t].float()).abs().max().item())
        worst_ref = max(worst_ref, np.abs(yt[:, 0].double().cpu().numpy() - y_ref[:, t]).max())
    assert worst <= 2e-2, worst
    assert worst_ref <= _oracle_tol(torch.bfloat16, y_ref[:, T0:]), worst_ref


def test_decode_from_one_token_fp32():
    B, T, D, H, es = 3, 20, 60, 4, 1.1                  # d = 15: 5 blocks, no leftover dims
    x, W = layer(43, B, T, D, H, "additive", dtype=torch.float32)
    m = make_module(W, D, H, es, "additive", torch.float32, DEV)
    y_full, _ = run_module(m, x, DEV, torch.float32)
    y_ref = R.forward_blocks(x, W, H, es, "additive")
    xt = torch.as_tensor(x).to(DEV, torch.float32)
    y0, st = m.prefill(xt[:, :1], capacity=64)
    assert (y0[:, 0] - y_full[:, 0]).abs().max().item() <= 2e-5
    for t in range(1, T):
        yt = m.decode_step(xt[:, t:t + 1], st)
        assert (yt[:, 0] - y_full[:, t]).abs().max().item() <= 2e-5, t
        assert np.abs(yt[:, 0].double().cpu().numpy() - y_ref[:, t]).max() <= 2e-5, t
    with pytest.raises(ValueError):
        st.t = st.capacity
        m.decode_step(xt[:, :1], st)
