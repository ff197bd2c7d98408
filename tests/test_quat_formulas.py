"""The quaternion formulas the kernels use (holo_common.h: qexp_skew, qmul,
qmat), restated in numpy and checked against the oracle's Rodrigues closed
form and matrix products. This pins the sign and component conventions of the
device code on the CPU; the GPU tests check the kernels themselves."""
from __future__ import annotations

import numpy as np

from oracle import holo_ref as R


def qexp_skew(a):
    a0, a1, a2 = a[..., 0], a[..., 1], a[..., 2]
    th2 = a0 * a0 + a1 * a1 + a2 * a2
    th = np.sqrt(th2)
    small = th2 < 1e-8
    ths = np.where(small, 1.0, th)
    c = np.where(small, 1 - 0.125 * th2, np.cos(0.5 * ths))
    s = np.where(small, 0.5 - th2 / 48.0, np.sin(0.5 * ths) / ths)
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
    rng = np.random.default_rng(0)
    for scale in (1e-6, 0.05, 0.7, 3.0):
        a = rng.standard_normal((400, 3)) * scale
        assert np.abs(qmat(qexp_skew(a)) - R.rodrigues(a)).max() < 1e-14


def test_hamilton_product_composes_rotations_left_to_right():
    rng = np.random.default_rng(1)
    a, b = rng.standard_normal((2, 300, 3))
    qa, qb = qexp_skew(a), qexp_skew(b)
    assert np.abs(qmat(qmul(qa, qb)) - R.rodrigues(a) @ R.rodrigues(b)).max() < 1e-14


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
    P_seq = R.prefix_blocks(R.rodrigues(a)[:, None])[:, 0]
    for c in range(nch):
        p = carry[c]
        for t in range(c * C, min(c * C + C, T)):
            assert np.abs(qmat(p) - P_seq[t]).max() < 1e-13
            if t + 1 < T:
                p = qmul(g[t], p)
