"""The exact path's backward oracle (oracle.holo_ref.exact_backward64: any
mask, causal mode with the wrap branch through the holonomy, inert mode)
against central differences of the exact-path forward (exact_attention64
through geometry_blocks, itself pinned to the brute-force arc walk of
core/attention.py:156-192 and to the reference's golden vectors), in
float64.

The gradient of L = <do, o(q, k, v, a)> is checked along random directions
of all inputs at once and of each input alone (q, k, v and the link
parameters a of all T edges, the closing edge included). Under the tril
mask the causal gradient must equal the tril backward oracle
(attention_backward64 + link_grad_from_cross, pinned against torch autograd
in tests/test_oracle_backward.py). Four planted mistakes (the holonomy's
torque dropped, Hol in place of Hol^T, the inert torque's sign and frame)
must each fail the difference check.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import holo_ref as R


def _case(seed, B, H, T, d, mask_kind, scale=0.6, a_scale=0.7):
    rng = np.random.default_rng(seed)
    m = 3 * (d // 3)
    q, k, v, do = (rng.standard_normal((B, H, T, d)) for _ in range(4))
    a = rng.standard_normal((B, H, T, m)) * a_scale
    mask = None
    if mask_kind == "random":
        mask = rng.random((T, T)) < 0.4
        mask[np.arange(T), rng.integers(0, T, T)] = True             # every row allows a key
    elif mask_kind == "ring":
        mask = R.ring_mask(T)
    elif mask_kind == "tril":
        mask = np.tril(np.ones((T, T), dtype=bool))
    return rng, (q, k, v, a), do, mask, scale


def _loss(args, do, mask, scale, mode):
    q, k, v, a = args
    P, Hol = R.geometry_blocks(a)
    return float((R.exact_attention64(q, k, v, P, Hol, scale, mask, mode) * do).sum())


def _fd_errors(args, do, mask, scale, mode, g, rng, eps=1e-5):
    """relative errors of the analytic directional derivatives: all inputs
    together (three directions), then each input alone."""
    names = ("dq", "dk", "dv", "da")
    out = []
    for sel in [None, None, None, 0, 1, 2, 3]:
        dirs = [rng.standard_normal(x.shape) if sel is None or sel == i else np.zeros_like(x)
                for i, x in enumerate(args)]
        lp = _loss([x + eps * u for x, u in zip(args, dirs)], do, mask, scale, mode)
        lm = _loss([x - eps * u for x, u in zip(args, dirs)], do, mask, scale, mode)
        fd = (lp - lm) / (2 * eps)
        an = sum(float((g[n] * u).sum()) for n, u in zip(names, dirs))
        out.append(abs(fd - an) / max(1.0, abs(fd)))
    return out


@pytest.mark.parametrize("mode", ["causal", "inert"])
@pytest.mark.parametrize("mask_kind", ["none", "random", "ring"])
@pytest.mark.parametrize("shape", [(1, 2, 7, 7), (2, 1, 12, 6), (1, 1, 1, 3)])
def test_exact_backward_equals_central_differences(mode, mask_kind, shape):
    B, H, T, d = shape                             # d = 7: two blocks and one unrotated dim
    rng, args, do, mask, scale = _case(31 + T, B, H, T, d, mask_kind)
    g = R.exact_backward64(*args, do, scale, mask, mode)
    errs = _fd_errors(args, do, mask, scale, mode, g, rng)
    assert max(errs) <= 1e-7, errs


def test_closing_edge_gradient():
    """The closing edge enters through the holonomy only: its gradient is
    non-zero in causal mode with wrap pairs open, zero in inert mode and
    under tril."""
    for mode, mask_kind, nonzero in (("causal", "none", True), ("inert", "none", False),
                                     ("causal", "tril", False)):
        _, args, do, mask, scale = _case(5, 1, 2, 9, 6, mask_kind)
        da = R.exact_backward64(*args, do, scale, mask, mode)["da"]
        assert (np.abs(da[:, :, -1]).max() > 1e-3) == nonzero, (mode, mask_kind)


def test_tril_mask_reduces_to_the_tril_backward():
    B, H, T, d = 2, 2, 11, 8
    _, (q, k, v, a), do, mask, scale = _case(9, B, H, T, d, "tril")
    g = R.exact_backward64(q, k, v, a, do, scale, mask, "causal")
    P, _ = R.geometry_blocks(a)
    nb = d // 3
    qh, kh, vh, doh = (R.apply_blocks_T(P, u) for u in (q, k, v, do))
    oh = R.causal_attention64(qh, kh, vh, scale)
    dqh, dkh, dvh = R.attention_backward64(qh, kh, vh, oh, doh, scale)
    b3 = lambda u: R._blocks3(u, nb)
    c = (np.cross(b3(oh), b3(doh)) + np.cross(b3(dqh), b3(qh)) + np.cross(b3(dkh), b3(kh))
         + np.cross(b3(dvh), b3(vh)))
    da = R.link_grad_from_cross(a.reshape(B, H, T, nb, 3), P, c).reshape(a.shape)
    ref = {"dq": R.apply_blocks(P, dqh), "dk": R.apply_blocks(P, dkh), "dv": R.apply_blocks(P, dvh), "da": da}
    for name, r in ref.items():
        assert np.abs(g[name] - r).max() <= 1e-12 * max(1.0, np.abs(r).max()), name


@pytest.mark.parametrize("plant,mode", [("no_holonomy_torque", "causal"), ("hol_not_transposed", "causal"),
                                        ("inert_torque_sign", "inert"), ("inert_torque_frame", "inert")])
def test_planted_mistakes_fail(plant, mode):
    rng, args, do, mask, scale = _case(21, 1, 2, 8, 6, "none")
    g = R.exact_backward64(*args, do, scale, mask, mode, plant=plant)
    assert max(_fd_errors(args, do, mask, scale, mode, g, rng)) > 1e-3
