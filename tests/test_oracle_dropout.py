"""Attention dropout in the oracle (kernel/attention_fast.py:160: an
nn.Dropout on the exact path's softmax weights; core/attention.py:190).

* philox4x32_10 against the published known-answer vectors of
  Philox4x32-10 (Random123's kat_vectors: zero, all-ones and pi-digit
  counters and keys), so the generator the kernels restate is the published
  one.
* dropout_keep: kept fraction within binomial bounds of 1 - p at several p,
  a row subset equal to the same rows of the full mask, p = 0 keeps all.
* exact_attention64 with a keep mask: all kept at drop_scale 1 gives the
  dropout-free output; the outputs of a mask and of its complement
  (drop_scale 1) sum to the dropout-free output in both modes and both
  branches, which fails if the mask acts on scores or on one branch only.
* exact_backward64 with a keep mask: the directional derivatives of
  <do, exact_attention64(..., keep, 1/(1-p))> by central differences (q, k,
  v and the link parameters of every edge), and two planted mistakes (the
  mask applied before the softmax; the weights' gradient left unscaled) fail.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import holo_ref as R

KAT = [  # (counter, key, Philox4x32-10 output)
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT)
def test_philox_known_answers(ctr, key, out):
    assert tuple(int(x) for x in R.philox4x32_10(np.array(ctr, dtype=np.uint32), key)) == out


def test_philox_vectorised_equals_single_calls():
    rng = np.random.default_rng(3)
    ctr = rng.integers(0, 2 ** 32, (5, 7, 4), dtype=np.uint64).astype(np.uint32)
    key = (0x12345678, 0x9ABCDEF0)
    full = R.philox4x32_10(ctr, key)
    for idx in [(0, 0), (4, 6), (2, 3)]:
        assert np.array_equal(full[idx], R.philox4x32_10(ctr[idx], key))


@pytest.mark.parametrize("p", [0.1, 0.3, 0.5, 0.9])
def test_keep_fraction_binomial(p):
    B, H, T = 2, 3, 300
    keep = R.dropout_keep(B, H, T, p, seed=0x5EED0000ABCD + int(p * 100), offset=7)
    n = keep.size
    frac = keep.mean()
    assert abs(frac - (1 - p)) <= 5 * math.sqrt(p * (1 - p) / n), frac
    # each of the four words of a counter, and both halves of the rows
    for e in range(4):
        sub = keep[..., e::4]
        assert abs(sub.mean() - (1 - p)) <= 5 * math.sqrt(p * (1 - p) / sub.size)


def test_keep_rows_and_edge_cases():
    B, H, T = 1, 2, 37
    full = R.dropout_keep(B, H, T, 0.4, seed=99, offset=3)
    rows = np.array([0, 5, 36])
    assert np.array_equal(R.dropout_keep(B, H, T, 0.4, seed=99, offset=3, rows=rows), full[:, :, rows])
    assert R.dropout_keep(B, H, T, 0.0, seed=99).all()
    assert not np.array_equal(full, R.dropout_keep(B, H, T, 0.4, seed=100, offset=3))
    assert not np.array_equal(full, R.dropout_keep(B, H, T, 0.4, seed=99, offset=4))
    assert not np.array_equal(full[:, 0], full[:, 1])       # heads draw apart
    assert R.dropout_threshold(0.0) == 0 and R.dropout_threshold(0.5) == 2 ** 31
    assert R.dropout_threshold(np.nextafter(np.float32(1), np.float32(0))) == 2 ** 32 - 2 ** 8


def _fwd_case(seed, B, H, T, d, mask_kind):
    rng = np.random.default_rng(seed)
    m = 3 * (d // 3)
    q, k, v = (rng.standard_normal((B, H, T, d)) for _ in range(3))
    a = rng.standard_normal((B, H, T, m)) * 0.7
    mask = R.ring_mask(T) if mask_kind == "ring" else None
    return q, k, v, a, mask


@pytest.mark.parametrize("mode", ["causal", "inert"])
@pytest.mark.parametrize("mask_kind", ["none", "ring"])
def test_complement_masks_sum_to_dropout_free(mode, mask_kind):
    B, H, T, d = 2, 2, 19, 7
    q, k, v, a, mask = _fwd_case(4, B, H, T, d, mask_kind)
    P, Hol = R.geometry_blocks(a)
    ref = R.exact_attention64(q, k, v, P, Hol, 0.5, mask, mode)
    keep = R.dropout_keep(B, H, T, 0.35, seed=1234)
    o1 = R.exact_attention64(q, k, v, P, Hol, 0.5, mask, mode, keep=keep, drop_scale=1.0)
    o2 = R.exact_attention64(q, k, v, P, Hol, 0.5, mask, mode, keep=~keep, drop_scale=1.0)
    assert np.abs(o1 + o2 - ref).max() <= 1e-12
    assert np.abs(o1 - ref).max() > 1e-2                   # the mask changes the output
    allk = R.exact_attention64(q, k, v, P, Hol, 0.5, mask, mode, keep=np.ones_like(keep), drop_scale=1.0)
    assert np.abs(allk - ref).max() <= 1e-14
    # scaling: drop_scale multiplies the output
    o3 = R.exact_attention64(q, k, v, P, Hol, 0.5, mask, mode, keep=keep, drop_scale=2.5)
    assert np.abs(o3 - 2.5 * o1).max() <= 1e-12


def _loss(args, do, mask, scale, mode, keep, ds):
    q, k, v, a = args
    P, Hol = R.geometry_blocks(a)
    return float((R.exact_attention64(q, k, v, P, Hol, scale, mask, mode, keep=keep, drop_scale=ds) * do).sum())


def _fd_errors(args, do, mask, scale, mode, keep, ds, g, rng, eps=1e-5):
    names = ("dq", "dk", "dv", "da")
    out = []
    for sel in [None, None, 0, 1, 2, 3]:
        dirs = [rng.standard_normal(x.shape) if sel is None or sel == i else np.zeros_like(x)
                for i, x in enumerate(args)]
        lp = _loss([x + eps * u for x, u in zip(args, dirs)], do, mask, scale, mode, keep, ds)
        lm = _loss([x - eps * u for x, u in zip(args, dirs)], do, mask, scale, mode, keep, ds)
        fd = (lp - lm) / (2 * eps)
        an = sum(float((g[n] * u).sum()) for n, u in zip(names, dirs))
        out.append(abs(fd - an) / max(1.0, abs(fd)))
    return out


@pytest.mark.parametrize("mode", ["causal", "inert"])
@pytest.mark.parametrize("mask_kind", ["none", "ring"])
def test_dropout_backward_equals_central_differences(mode, mask_kind):
    B, H, T, d, p = 1, 2, 11, 7, 0.3
    q, k, v, a, mask = _fwd_case(17, B, H, T, d, mask_kind)
    rng = np.random.default_rng(18)
    do = rng.standard_normal(q.shape)
    keep = R.dropout_keep(B, H, T, p, seed=77, offset=1)
    ds = 1.0 / (1.0 - p)
    g = R.exact_backward64(q, k, v, a, do, 0.6, mask, mode, keep=keep, drop_scale=ds)
    errs = _fd_errors((q, k, v, a), do, mask, 0.6, mode, keep, ds, g, rng)
    assert max(errs) <= 1e-7, errs
    g0 = R.exact_backward64(q, k, v, a, do, 0.6, mask, mode)
    assert np.abs(g["dv"] - g0["dv"]).max() > 1e-2         # dropout changes the gradient


@pytest.mark.parametrize("plant", ["dropout_before_softmax", "dropout_grad_unscaled"])
def test_dropout_planted_mistakes_fail(plant):
    B, H, T, d, p = 1, 2, 10, 6, 0.4
    q, k, v, a, mask = _fwd_case(23, B, H, T, d, "none")
    rng = np.random.default_rng(24)
    do = rng.standard_normal(q.shape)
    keep = R.dropout_keep(B, H, T, p, seed=5)
    ds = 1.0 / (1.0 - p)
    g = R.exact_backward64(q, k, v, a, do, 0.6, mask, "causal", plant=plant, keep=keep, drop_scale=ds)
    assert max(_fd_errors((q, k, v, a), do, mask, 0.6, "causal", keep, ds, g, rng)) > 1e-3
