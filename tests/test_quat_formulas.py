"""The quaternion formulas the kernels use (holo_common.h: qexp_skew, qmul,
qmat), restated in numpy and checked against the oracle's Rodrigues closed
form and matrix products. This pins the sign and component conventions of the
device code on the CPU; the GPU tests check the kernels themselves."""
from __future__ import annotations

import numpy as np

from oracle import holo_ref as R


def qexp_skew(a):
    """Below th = 1 the device code evaluates cos(th/2) and sin(th/2)/th as
    Taylor series in th^2 (Horner, through th^8); above, the closed form."""
    a0, a1, a2 = a[..., 0], a[..., 1], a[..., 2]
    th2 = a0 * a0 + a1 * a1 + a2 * a2
    th = np.sqrt(th2)
    small = th2 < 1.0
    ths = np.where(small, 1.0, th)
    cs = 1 + th2 * (-1 / 8 + th2 * (1 / 384 + th2 * (-1 / 46080 + th2 * (1 / 10321920))))
    ss = 0.5 + th2 * (-1 / 48 + th2 * (1 / 3840 + th2 * (-1 / 645120 + th2 * (1 / 185794560))))
    c = np.where(small, cs, np.cos(0.5 * ths))
    s = np.where(small, ss, np.sin(0.5 * ths) / ths)
    return np.stack([c, -a2 * s, a1 * s, -a0 * s], -1)


def qmul(a, b):
    aw, ax, ay, az = np.moveaxis(a, -1, 0)
    bw, bx, by, bz = np.moveaxis(b, -1, 0)
    return np.stack([aw * bw - ax * bx - ay * by - az * bz,
                     aw * bx + ax * bw + ay * bz - az * by,
                     aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw], -1)


def qmat(q):
    w, x, y, z = np.moveaxis(q, -1, 0)
    inv = 1.0 / (w * w + x * x + y * y + z * z)
    return np.stack([
        np.stack([(w * w + x * x - y * y - z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        np.stack([2 * (x * y + w * z), (w * w - x * x + y * y - z * z), 2 * (y * z - w * x)], -1),
        np.stack([2 * (x * z - w * y), 2 * (y * z + w * x), (w * w - x * x - y * y + z * z)], -1),
    ], -2) * inv[..., None, None]


def test_quaternion_exp_is_rodrigues():
    """Within the series' truncation below th = 1 (omitted terms < 3e-10 of
    the coefficients, so < 2e-9 per matrix entry), exactly the closed form above."""
    rng = np.random.default_rng(0)
    for scale in (1e-6, 0.05, 0.7, 3.0):
        a = rng.standard_normal((400, 3)) * scale
        assert np.abs(qmat(qexp_skew(a)) - R.rodrigues(a)).max() < 2e-9
    big = rng.standard_normal((400, 3)) * 3.0
    big = big[np.sum(big * big, -1) >= 1.0]
    assert np.abs(qmat(qexp_skew(big)) - R.rodrigues(big)).max() < 1e-14


def test_link_exp_series_coefficients():
    """cos(th/2) and sin(th/2)/th from the series against the closed form on
    [0, 1): truncation below 3e-10, largest at th -> 1."""
    th = np.linspace(1e-3, 1.0, 5001)[:-1]
    q = qexp_skew(np.stack([np.zeros_like(th), np.zeros_like(th), th], -1))   # w = (-th, 0, 0)
    assert np.abs(q[:, 0] - np.cos(th / 2)).max() < 3e-10
    assert np.abs(-q[:, 1] / th - np.sin(th / 2) / th).max() < 3e-10


def test_hamilton_product_composes_rotations_left_to_right():
    rng = np.random.default_rng(1)
    a, b = rng.standard_normal((2, 300, 3))
    qa, qb = qexp_skew(a), qexp_skew(b)
    assert np.abs(qmat(qmul(qa, qb)) - qmat(qa) @ qmat(qb)).max() < 1e-14


def test_homogeneous_matrix_ignores_quaternion_norm():
    rng = np.random.default_rng(2)
    q = qexp_skew(rng.standard_normal((100, 3)))
    assert np.abs(qmat(q * 1.37) - qmat(q)).max() < 1e-15


def test_chunked_quaternion_scan_equals_sequential_products():
    """Chunk totals, exclusive carries and re-anchored intra-chunk products
    (the three scan launches) reproduce P_{t+1} = G_t P_t."""
    rng = np.random.default_rng(3)
    T, C = 300, 64
    a = rng.standard_normal((T - 1, 3)) * 0.4
    g = qexp_skew(a)
    nch = (T + C - 1) // C
    tot = []
    for c in range(nch):
        acc = np.array([1.0, 0, 0, 0])
        for t in range(c * C, min(c * C + C, T - 1)):
            acc = qmul(g[t], acc)
        tot.append(acc)
    carry, cur = [], np.array([1.0, 0, 0, 0])
    for c in range(nch):
        carry.append(cur)
        cur = qmul(tot[c], cur)
    P_seq = R.prefix_blocks(qmat(g)[:, None])[:, 0]            # the links' own matrices, composed in order
    for c in range(nch):
        p = carry[c]
        for t in range(c * C, min(c * C + C, T)):
            assert np.abs(qmat(p) - P_seq[t]).max() < 1e-13
            if t + 1 < T:
                p = qmul(g[t], p)
