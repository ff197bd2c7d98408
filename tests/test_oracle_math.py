"""Mathematical pins of the oracle that do not depend on the reference code:
closed forms, library routines, invariants and brute force at tiny sizes."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import holo_ref as R
from tests._util import layer


def _skew3(a):
    a0, a1, a2 = a[..., 0], a[..., 1], a[..., 2]
    z = np.zeros_like(a0)
    return np.stack([np.stack([z, a0, a1], -1), np.stack([-a0, z, a2], -1),
                     np.stack([-a1, -a2, z], -1)], -2)


@pytest.mark.parametrize("scale", [1e-7, 1e-3, 0.12, 1.0, 3.0, 10.0])
def test_rodrigues_is_the_matrix_exponential(scale):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((500, 3)) * scale
    G = R.rodrigues(a)
    ref = torch.linalg.matrix_exp(torch.as_tensor(_skew3(a))).numpy()
    assert np.abs(G - ref).max() < 1e-13 * max(1.0, scale)


def test_rodrigues_invariants():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((1000, 3)) * 2.0
    G = R.rodrigues(a)
    eye = np.eye(3)
    assert np.abs(np.swapaxes(G, -1, -2) @ G - eye).max() < 1e-14
    assert np.abs(np.linalg.det(G) - 1).max() < 1e-14
    assert np.abs(G @ R.rodrigues(-a) - eye).max() < 1e-14          # exp(A) exp(-A) = I
    assert np.array_equal(R.rodrigues(np.zeros((1, 3)))[0], eye)     # exp(0) = I
    # angle pi about an axis: R = 2 n n^T - I
    n = np.array([1.0, -2.0, 2.0]) / 3.0
    w = np.pi * n                              # w = (-a2, a1, -a0)
    Gp = R.rodrigues(np.array([-w[2], w[1], -w[0]]))
    assert np.abs(Gp - (2 * np.outer(n, n) - eye)).max() < 1e-14
    # continuity across the small-angle switch
    th = np.array([0.99e-4, 1.01e-4])
    Gs = R.rodrigues(np.stack([th, np.zeros(2), np.zeros(2)], -1))
    assert abs(Gs[0, 0, 1] - math.sin(th[0])) < 1e-16 and abs(Gs[1, 0, 1] - math.sin(th[1])) < 1e-16


def test_skew_layout_and_block_embedding():
    d = 9
    v = torch.arange(1, d * (d - 1) // 2 + 1, dtype=torch.float64)
    A = R.skew_from_vec(v, d)
    assert torch.equal(A, -A.T)
    k = 0
    for i in range(d):                          # row-major upper triangle
        for j in range(i + 1, d):
            assert A[i, j] == v[k]
            k += 1
    mp = R.block_to_dense_map(d)
    assert list(mp[:3]) == [R.dense_index(0, 1, d), R.dense_index(0, 2, d), R.dense_index(1, 2, d)]
    assert list(mp) == [0, 1, 8, 21, 22, 26, 33, 34, 35]
    assert R.block_to_dense_map(96)[-3:].tolist() == [4557, 4558, 4559]
    assert R.block_to_dense_map(96)[:3].tolist() == [0, 1, 95]
    with pytest.raises(ValueError):
        R.skew_from_vec(torch.zeros(5), 4)


def test_prefix_products_brute_force():
    rng = np.random.default_rng(2)
    G = R.rodrigues(rng.standard_normal((2, 7, 4, 3)))      # (B=2, T-1=7, nb=4)
    P = R.prefix_blocks(G)
    assert np.array_equal(P[:, 0], np.broadcast_to(np.eye(3), (2, 4, 3, 3)))
    for t in range(1, 8):
        M = np.broadcast_to(np.eye(3), (2, 4, 3, 3)).copy()
        for s in range(t):
            M = G[:, s] @ M
        assert np.abs(P[:, t] - M).max() < 1e-14


def test_block_oracle_equals_chunked_oracle_fp64():
    for lm in ("additive", "interaction"):
        x, W = layer(31, 2, 130, 60, 4, lm, dtype=torch.float64)      # d = 15, three key blocks
        Wt = {k: torch.as_tensor(v) for k, v in W.items()}
        y_c = R.forward_chunked(torch.as_tensor(x), Wt, 4, 0.9, lm).numpy()
        y_b = R.forward_blocks(x, W, 4, 0.9, lm)
        assert np.abs(y_c - y_b).max() < 1e-12


def test_flat_connection_reduces_to_causal_sdpa():
    """edge_scale = 0: every rotation is the identity and the layer is plain
    causal softmax attention (PDF Theorem 1)."""
    B, T, D, H = 2, 50, 48, 4
    x, W = layer(32, B, T, D, H, dtype=torch.float64)
    y = R.forward_blocks(x, W, H, 0.0)
    d = D // H
    xt = torch.as_tensor(x)
    qkv = (xt @ torch.as_tensor(W["qkv.weight"]).T).view(B, T, H, 3 * d).transpose(1, 2)
    o = torch.nn.functional.scaled_dot_product_attention(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:],
                                                         is_causal=True)
    y_ref = (o.transpose(1, 2).reshape(B, T, D) @ torch.as_tensor(W["out.weight"]).T).numpy()
    assert np.abs(y - y_ref).max() < 1e-12


def test_global_gauge_rotation_cancels():
    """Replacing every prefix P_t by P_t R0 for a fixed block rotation R0 (a
    change of the frame at token 0, PDF Theorem 3) leaves the output unchanged:
    q^.k^ and P_i sum p v^ only involve P_i P_j^T."""
    B, T, D, H = 1, 40, 36, 2
    x, W = layer(33, B, T, D, H, dtype=torch.float64)
    y, parts = R.forward_blocks(x, W, H, 0.8, return_parts=True)
    rng = np.random.default_rng(3)
    R0 = R.rodrigues(rng.standard_normal((H, 1, parts["P"].shape[3], 3)))
    P2 = parts["P"] @ R0[None]
    qh, kh, vh = (R.apply_blocks_T(P2, parts[n]) for n in ("q", "k", "v"))
    oh = R.causal_attention64(qh, kh, vh, 1.0 / math.sqrt(D // H))
    o = R.apply_blocks(P2, oh).transpose(0, 2, 1, 3).reshape(B, T, D)
    assert np.abs(o @ W["out.weight"].T - y).max() < 1e-12


def test_causal_prefix_consistency_oracle():
    B, T, D, H, s = 1, 60, 36, 2, 23
    x, W = layer(34, B, T, D, H, dtype=torch.float64)
    y1 = R.forward_blocks(x, W, H, 0.8)
    x2 = x.copy()
    x2[:, s:] = -3.0 * x2[:, s:]
    y2 = R.forward_blocks(x2, W, H, 0.8)
    assert np.abs(y1[:, :s] - y2[:, :s]).max() < 1e-13
    assert np.abs(y1[:, s:] - y2[:, s:]).max() > 1e-3


def test_prefix_transport_is_the_arc_walk():
    """forward_blocks (prefix products) equals the O(L^3) arc walk at small L."""
    x, W = layer(35, 2, 9, 24, 2, dtype=torch.float64)
    assert np.abs(R.forward_blocks(x, W, 2, 1.3) - R.forward_arc_walk(x, W, 2, 1.3)).max() < 1e-12


def test_attention_rows_equal_full_causal_attention():
    """oracle.attention_rows64 (the parity-bar tests' row-wise oracle) against
    the rows of causal_attention64 and against torch's causal
    scaled_dot_product_attention (float64), at unsorted and repeated rows,
    row 0 (one key) and the last row; an off-by-one causal mask (query i sees
    keys 0..i-1, row 0 dropped) must fail the comparison."""
    rng = np.random.default_rng(5)
    qh, kh, vh = (rng.standard_normal((2, 3, 150, 12)) for _ in range(3))
    scale = 1.0 / math.sqrt(12)
    rows = np.array([149, 0, 37, 37, 64, 1, 148])
    got = R.attention_rows64(qh, kh, vh, scale, rows)
    full = R.causal_attention64(qh, kh, vh, scale)
    np.testing.assert_allclose(got, full[..., rows, :], rtol=0, atol=1e-12)
    sdpa = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(u) for u in (qh, kh, vh)), is_causal=True, scale=scale).numpy()
    np.testing.assert_allclose(got, sdpa[..., rows, :], rtol=0, atol=1e-12)
    # planted mistake: strict causality (keys j < i) on rows >= 1
    r1 = rows[rows > 0]
    s = np.matmul(qh[..., r1, :], np.swapaxes(kh, -1, -2)) * scale
    s = np.where(r1[:, None] > np.arange(150)[None, :], s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    wrong = np.matmul(p / p.sum(axis=-1, keepdims=True), vh)
    assert np.abs(wrong - R.attention_rows64(qh, kh, vh, scale, r1)).max() > 1e-3
