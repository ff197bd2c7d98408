"""The C ABI from a C caller with no PyTorch (tests/c/abi_smoke.c, built by
__graft_entry__.build()): HIP-runtime allocations, holo_geom_scan_fwd +
holo_attn_fwd (causal, tril) and holo_attn_masked_fwd (ring mask), fp32,
against the float64 oracle on the same inputs; the driver also checks the
error path (status code and message of a bad call).

The driver also runs the documented C binding example
(tests/c/integration_example.c: the bf16 path with fp16 operands, o in fp32)
on the same q, k, v rounded to bf16.

Tolerance (written in the test): fp32 max-abs <= 2e-5 (the fp32 bar; the ring
mask's wrap branch carries the holonomy, a product of all T links); the bf16
path's per-head o max-abs <= 2e-3 against the oracle on the bf16-rounded
inputs (the bf16 bar).
"""
from __future__ import annotations

import math
import os
import subprocess

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import build as _build
from oracle import holo_ref as R

pytestmark = pytest.mark.gpu


def test_c_caller_matches_oracle(tmp_path):
    if not os.path.exists(_build.C_SMOKE_BIN):
        pytest.fail(f"{_build.C_SMOKE_BIN} not built (run __graft_entry__.build())")
    B, T, H, d, es = 2, 150, 2, 48, 0.8
    m = 3 * (d // 3)
    rng = np.random.default_rng(11)
    q, k, v = (rng.standard_normal((B, T, H, d)).astype(np.float32) for _ in range(3))
    gq, gk = (rng.standard_normal((B, T, H, m)).astype(np.float32) for _ in range(2))
    for name, arr in (("q", q), ("k", k), ("v", v), ("gq", gq), ("gk", gk)):
        arr.tofile(tmp_path / f"{name}.f32")
    print(f"C ABI driver B={B} T={T} H={H} d={d}", flush=True)
    r = subprocess.run([_build.C_SMOKE_BIN, str(tmp_path), str(B), str(T), str(H), str(d), str(es)],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    o_tril = np.fromfile(tmp_path / "o_tril.f32", dtype=np.float32).reshape(B, T, H, d).astype(np.float64)
    o_ring = np.fromfile(tmp_path / "o_ring.f32", dtype=np.float32).reshape(B, T, H, d).astype(np.float64)

    f64 = lambda a: a.astype(np.float64).transpose(0, 2, 1, 3)          # (B, H, T, .)
    a = es * (f64(gq) + np.roll(f64(gk), -1, axis=2))                      # a_t = es (gq_t + gk_{t+1 mod T})
    P, Hol = R.geometry_blocks(a)
    qq, kk, vv = f64(q), f64(k), f64(v)
    scale = 1.0 / math.sqrt(d)
    ref_tril = R.apply_blocks(P, R.causal_attention64(R.apply_blocks_T(P, qq), R.apply_blocks_T(P, kk),
                                                      R.apply_blocks_T(P, vv), scale))
    ref_ring = R.exact_attention64(qq, kk, vv, P, Hol, scale, R.ring_mask(T), "causal")
    err_tril = np.abs(o_tril - ref_tril.transpose(0, 2, 1, 3)).max()
    err_ring = np.abs(o_ring - ref_ring.transpose(0, 2, 1, 3)).max()
    o_bf16 = np.fromfile(tmp_path / "o_bf16.f32", dtype=np.float32).reshape(B, T, H, d).astype(np.float64)
    rb = lambda a: torch.as_tensor(a).to(torch.bfloat16).double().numpy()
    qb, kb, vb = (rb(u) for u in (qq, kk, vv))
    ref_bf16 = R.apply_blocks(P, R.causal_attention64(R.apply_blocks_T(P, qb), R.apply_blocks_T(P, kb),
                                                      R.apply_blocks_T(P, vb), scale))
    err_bf16 = np.abs(o_bf16 - ref_bf16.transpose(0, 2, 1, 3)).max()
    print(f"max-abs: tril {err_tril:.3e}, ring {err_ring:.3e}, bf16 binding {err_bf16:.3e}")
    assert err_tril <= 2e-5 and err_ring <= 2e-5
    assert err_bf16 <= 2e-3
