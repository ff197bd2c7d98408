"""The hand-written projection GEMM (holo_qkvg_proj_fwd) against float64
products of the same bf16 inputs.

Bounds (written in the test): the bf16 x bf16 products are exact in fp32 and
the K-term sums are accumulated in fp32, so any summation order is within
K * 2^-24 * sum_c |x_c w_c|; the q/k/v outputs are then rounded once to bf16
(unit roundoff 2^-8: 8 significant bits). The generator sum g_t = x_t W_gq^T + x_{t+1} W_gk^T has 2K
terms and is stored in fp32.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import kernels
from tests._util import layer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _check(B, T, D, H, seed, rows=None):
    x, W = layer(seed, B, T, D, H, dtype=torch.bfloat16)
    xt = torch.as_tensor(x).to(DEV, torch.bfloat16)
    wq, wg0, wg1 = (torch.as_tensor(W[k]).to(DEV, torch.bfloat16).contiguous()
                    for k in ("qkv.weight", "gqproj.weight", "gkproj.weight"))
    qkv, g = kernels.qkvg_projection(xt, wq, wg0, wg1)
    torch.cuda.synchronize()
    xs = x.reshape(B * T, D)
    xn = np.roll(x, -1, axis=1).reshape(B * T, D)          # x_{(t+1) mod T} of the same sequence
    r = np.arange(B * T) if rows is None else np.asarray(rows)
    Wq, Wg0, Wg1 = (np.asarray(W[k]) for k in ("qkv.weight", "gqproj.weight", "gkproj.weight"))
    ref_q = xs[r] @ Wq.T
    ref_g = xs[r] @ Wg0.T + xn[r] @ Wg1.T
    mag_q = np.abs(xs[r]) @ np.abs(Wq).T
    mag_g = np.abs(xs[r]) @ np.abs(Wg0).T + np.abs(xn[r]) @ np.abs(Wg1).T
    got_q = qkv.reshape(B * T, -1)[torch.as_tensor(r, device=DEV)].double().cpu().numpy()
    got_g = g.reshape(B * T, -1)[torch.as_tensor(r, device=DEV)].double().cpu().numpy()
    bq = 2.0 ** -8 * np.abs(ref_q) + (1 + 2.0 ** -8) * D * 2.0 ** -24 * mag_q
    bg = 2 * D * 2.0 ** -24 * mag_g
    eq, eg = np.abs(got_q - ref_q), np.abs(got_g - ref_g)
    print(f"B={B} T={T} D={D} H={H}: qkv max err {eq.max():.3e} (err/bound {(eq / bq).max():.3f}), "
          f"g max err {eg.max():.3e} (err/bound {(eg / bg).max():.3f})")
    assert np.all(eq <= bq) and np.all(eg <= bg)


def test_qkvg_cfg2_rows():
    """Config 2's shape (M = 32768, K = 1536, 4608 + 1536 outputs): batch row 0
    whole, and the last two tokens of every sequence (the wrap to token 0)."""
    B, T, D, H = 16, 2048, 1536, 16
    rows = np.concatenate([np.arange(T)] + [[b * T + T - 2, b * T + T - 1] for b in range(1, B)])
    _check(B, T, D, H, 51, rows)


@pytest.mark.parametrize("B,T,D,H", [(3, 100, 128, 4), (5, 1, 128, 4), (2, 257, 192, 4), (1, 300, 384, 4)])
def test_qkvg_ragged_shapes(B, T, D, H):
    """M and the output widths not multiples of the 256 x 256 tile; T = 1
    (every token's successor is itself)."""
    _check(B, T, D, H, 52)
