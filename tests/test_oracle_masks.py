"""The oracle's exact path for every mode and mask (oracle.holo_ref.
exact_attention64 / forward_exact_blocks, restating kernel/attention_fast.py:
84-166) pinned against independent formulations:

* the O(L^3) arc walk of the definition (core/attention.py:156-192: compose
  the edge rotations along the ring arc, inert mode the endpoint transport
  C_i^T C_j), for no mask, the ring mask, random masks and tril;
* forward_blocks (itself pinned by the reference's golden vectors) under
  causal + tril;
* the flat connection (edge_scale = 0: every transport is the identity), where
  both modes are torch's scaled_dot_product_attention with the same mask;
* planted mistakes (Hol for Hol^T, P for P^T) that the checks must catch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import holo_ref as R
from tests._util import layer


def _random_mask(T, seed, p=0.5):
    m = np.random.default_rng(seed).random((T, T)) < p
    m[np.arange(T), np.arange(T)] = True           # every row allows something
    return m


def test_ring_mask_matches_its_definition():
    T = 7
    ref = np.zeros((T, T), dtype=bool)
    for i in range(T):                              # core/utils.py:70-74
        for j in (i, (i - 1) % T, (i + 1) % T):
            ref[i, j] = True
    assert np.array_equal(R.ring_mask(T), ref)
    assert R.ring_mask(T)[0, T - 1] and R.ring_mask(T)[T - 1, 0]


@pytest.mark.parametrize("lm", ["additive", "interaction"])
def test_exact_path_under_tril_is_forward_blocks(lm):
    x, W = layer(41, 2, 37, 48, 4, lm, dtype=torch.float64)
    tril = np.tril(np.ones((37, 37), dtype=bool))
    y = R.forward_exact_blocks(x, W, 4, 0.9, lm, mask=tril, mode="causal")
    assert np.abs(y - R.forward_blocks(x, W, 4, 0.9, lm)).max() < 1e-12


@pytest.mark.parametrize("mode", ["causal", "inert"])
@pytest.mark.parametrize("mask_kind", ["none", "ring", "random", "tril"])
def test_exact_path_is_the_arc_walk(mode, mask_kind):
    B, T, D, H, es = 2, 9, 24, 2, 1.3
    x, W = layer(42, B, T, D, H, dtype=torch.float64)
    mask = {"none": None, "ring": R.ring_mask(T), "random": _random_mask(T, 5),
            "tril": np.tril(np.ones((T, T), dtype=bool))}[mask_kind]
    y = R.forward_exact_blocks(x, W, H, es, mask=mask, mode=mode)
    y_walk = R.forward_arc_walk(x, W, H, es, mask=mask, mode=mode)
    assert np.abs(y - y_walk).max() < 1e-12


def test_modes_differ_off_the_flat_connection():
    """Under tril the causal transport is P_i P_j^T and the inert one P_i^T P_j:
    they agree only when the rotations commute (here they do not)."""
    x, W = layer(43, 1, 12, 24, 2, dtype=torch.float64)
    tril = np.tril(np.ones((12, 12), dtype=bool))
    yc = R.forward_exact_blocks(x, W, 2, 1.3, mask=tril, mode="causal")
    yi = R.forward_exact_blocks(x, W, 2, 1.3, mask=tril, mode="inert")
    assert np.abs(yc - yi).max() > 1e-3


@pytest.mark.parametrize("mode", ["causal", "inert"])
def test_flat_connection_is_sdpa_with_the_mask(mode):
    B, T, D, H = 2, 40, 48, 4
    d = D // H
    x, W = layer(44, B, T, D, H, dtype=torch.float64)
    mask = _random_mask(T, 6, p=0.3)
    y = R.forward_exact_blocks(x, W, H, 0.0, mask=mask, mode=mode)
    qkv = (torch.as_tensor(x) @ torch.as_tensor(W["qkv.weight"]).T).view(B, T, H, 3 * d).transpose(1, 2)
    o = torch.nn.functional.scaled_dot_product_attention(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:],
                                                         attn_mask=torch.as_tensor(mask))
    y_ref = (o.transpose(1, 2).reshape(B, T, D) @ torch.as_tensor(W["out.weight"]).T).numpy()
    assert np.abs(y - y_ref).max() < 1e-12


def test_row_with_no_allowed_key_is_nan():
    """The reference masks with -inf and applies torch.softmax, which gives NaN
    for a row of -inf only (kernel/attention_fast.py:154-158)."""
    assert torch.isnan(torch.softmax(torch.full((3,), -math.inf), -1)).all()
    B, T, D, H = 1, 10, 24, 2
    x, W = layer(45, B, T, D, H, dtype=torch.float64)
    mask = _random_mask(T, 7)
    mask[4] = False
    for mode in ("causal", "inert"):
        y = R.forward_exact_blocks(x, W, H, 0.7, mask=mask, mode=mode)
        assert np.isnan(y[:, 4]).all() and np.isfinite(np.delete(y, 4, axis=1)).all()
        assert np.isnan(R.forward_arc_walk(x, W, H, 0.7, mask=mask, mode=mode)[:, 4]).all()


def test_planted_transport_mistakes_are_caught():
    """Hol^T for Hol in the wrap branch, or P^T for P in inert mode, moves the
    output far from the arc walk, so the agreement above pins both sides."""
    B, T, D, H, es = 1, 8, 24, 2, 1.3
    x, W = layer(46, B, T, D, H, dtype=torch.float64)
    _, parts = R.forward_exact_blocks(x, W, H, es, mask=None, mode="causal", return_parts=True)
    q, k, v, P, Hol = (parts[n] for n in ("q", "k", "v", "P", "Hol"))
    d = D // H
    walk_c = R.forward_arc_walk(x, W, H, es, mask=None, mode="causal")
    walk_i = R.forward_arc_walk(x, W, H, es, mask=None, mode="inert")
    wout = W["out.weight"].T

    def y_of(o):
        return o.transpose(0, 2, 1, 3).reshape(B, T, D) @ wout

    good_c = y_of(R.exact_attention64(q, k, v, P, Hol, 1 / math.sqrt(d), None, "causal"))
    bad_c = y_of(R.exact_attention64(q, k, v, P, np.swapaxes(Hol, -1, -2), 1 / math.sqrt(d), None, "causal"))
    assert np.abs(good_c - walk_c).max() < 1e-12 and np.abs(bad_c - walk_c).max() > 1e-3
    bad_i = y_of(R.exact_attention64(q, k, v, np.swapaxes(P, -1, -2), Hol, 1 / math.sqrt(d), None, "inert"))
    assert np.abs(bad_i - walk_i).max() > 1e-3
