"""The float64 reference of the config 5 decode bar test
(tests/test_gpu_zy_config_bars.py::decode_oracle), which assembles each
decoded token's o_t from the prefix's projections and the per-step inputs
the decode wrappers received, against the full-sequence oracle on the same
inputs: equal to rounding (1e-12). An off-by-one in the captured link
parameters (gk of token t+1 instead of t) must fail."""
from __future__ import annotations

import math

import numpy as np

from oracle import holo_ref as R
from tests.test_gpu_zy_config_bars import decode_oracle


def _full_sequence(q, k, v, gq, gk, es, rows):
    bh = lambda u: u.transpose(0, 2, 1, 3)
    a = es * (bh(gq) + np.roll(bh(gk), -1, axis=2))
    P, _ = R.geometry_blocks(a)
    qh, kh, vh = (R.apply_blocks_T(P, bh(u)) for u in (q, k, v))
    oh = R.attention_rows64(qh, kh, vh, 1.0 / math.sqrt(q.shape[-1]), rows)
    return R.apply_blocks(P[:, :, rows], oh)


def test_decode_oracle_equals_full_sequence_oracle():
    rng = np.random.default_rng(0)
    b, T0, n, H, d, es = 2, 70, 10, 2, 12, 0.9
    T = T0 + n
    q, k, v = (rng.standard_normal((b, T, H, d)) for _ in range(3))
    gq, gk = (rng.standard_normal((b, T, H, d)) for _ in range(2))
    prefix = tuple(u[:, :T0] for u in (q, k, v, gq, gk))
    steps = [(t, q[:, t], k[:, t], v[:, t], gq[:, t - 1], gk[:, t]) for t in range(T0, T)]
    rows = np.array([T0, T0 + 1, T - 1])
    refs = decode_oracle(prefix, steps, es, list(rows))
    full = _full_sequence(q, k, v, gq, gk, es, rows)
    for i, t in enumerate(rows):
        assert np.abs(refs[int(t)] - full[:, :, i]).max() < 1e-12
    # planted: the link parameters of the wrong token
    bad = [(t, q[:, t], k[:, t], v[:, t], gq[:, t - 1], gk[:, min(t + 1, T - 1)]) for t in range(T0, T)]
    refs_bad = decode_oracle(prefix, bad, es, list(rows))
    assert max(np.abs(refs_bad[int(t)] - full[:, :, i]).max() for i, t in enumerate(rows)) > 1e-3
