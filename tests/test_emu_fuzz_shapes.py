"""Seeded random shapes on the CPU execution of the kernels (tests/emu):
batch, heads, sequence length, head dimension (every value 3..96, so every
padded width and leftover-dims case), masks, modes, operand types and
dropout probabilities drawn from a fixed generator, so the set is the same on
every run. Each case runs one entry point chain through the C ABI against
the float64 oracle, with the bounds checks of tests/test_emu_kernels.py and
its tolerances (the check functions are that file's): the scan + causal
attention (fp32 and fp16 operands), the exact path (both modes, five masks),
the fused backward, the exact path's training pair with and without
attention dropout, incremental decode, the projection GEMM and the fused
interaction generator's two GEMMs.

The fixed shapes of the other emulation tests follow the GPU tests; these
add the shapes in between, where index arithmetic on partial tiles, padded
rows and head strides would show an error that the regular shapes hide."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tests.emu import build_emu, jobs
from tests.test_emu_kernels import (BF16, F16, F32, S16, _bwd, _decode, _drop, _edge, _fp32_scan_attn, _gemm, _h16,
                                    _masked, _mbwd, _norm)

pytestmark = pytest.mark.skipif(not (os.path.exists(build_emu.CLANG) and os.path.exists(build_emu.ASAN_RT)),
                                reason="the CPU emulation needs ROCm's clang and its AddressSanitizer runtime")

_rng = np.random.default_rng(20261202)
FUZZ = []          # (id, case, params, check)


def _shape(tmax=300):
    return (int(_rng.integers(1, 4)), int(_rng.integers(1, tmax + 1)), int(_rng.choice([1, 2, 3, 5])),
            int(_rng.integers(3, 97)))


for i in range(8):
    B, T, H, d = _shape()
    es = float(_rng.uniform(0.05, 1.5))
    FUZZ.append((f"scan_attn_f32_{i}_B{B}_T{T}_H{H}_d{d}", "scan_attn", dict(B=B, T=T, H=H, d=d, es=es, seed=100 + i),
                 _fp32_scan_attn))
for i in range(6):
    B, T, H, d = _shape()
    FUZZ.append((f"scan_attn_f16_{i}_B{B}_T{T}_H{H}_d{d}", "scan_attn",
                 dict(B=B, T=T, H=H, d=d, io=BF16, op=F16, pf=S16, out=F32, es=0.5, seed=200 + i), _h16(F32)))
for i in range(10):
    B, T, H, d = _shape()
    mode = str(_rng.choice(["causal", "inert"]))
    mask = str(_rng.choice(["none", "ring", "random", "tril", "empty_row"]))
    io = F32 if i % 2 == 0 else BF16
    FUZZ.append((f"masked_{i}_{mode}_{mask}_io{io}_B{B}_T{T}_H{H}_d{d}", "masked",
                 dict(B=B, T=T, H=H, d=d, io=io, mode=mode, mask=mask, pf=0 if io == F32 else S16, seed=300 + i),
                 _masked(io)))
for i in range(5):
    B, T, H, d = _shape(200)
    gen = i % 2
    FUZZ.append((f"bwd_f32_{i}_gen{gen}_B{B}_T{T}_H{H}_d{d}", "bwd",
                 dict(B=B, T=T, H=H, d=d, es=0.9, gen=gen, seed=400 + i), _bwd(F32)))
for i in range(10):
    B, T, H, d = _shape(200)
    mode = str(_rng.choice(["causal", "inert"]))
    mask = str(_rng.choice(["none", "ring", "random", "tril"]))
    wrap = mode == "causal" and mask != "tril" and T > 1
    params = dict(B=B, T=T, H=H, d=d, mode=mode, mask=mask, io=F32, es=0.9, gen=i % 2, seed=500 + i)
    if i % 2:
        p = round(float(_rng.uniform(0.05, 0.6)), 3)
        params["drop"] = {"p": p, "seed": int(_rng.integers(0, 2 ** 63)), "offset": int(_rng.integers(0, 2 ** 32))}
        FUZZ.append((f"dropout_{i}_{mode}_{mask}_B{B}_T{T}_H{H}_d{d}_p{p}", "masked_bwd", params, _drop(F32, wrap, p)))
    else:
        FUZZ.append((f"masked_bwd_{i}_{mode}_{mask}_B{B}_T{T}_H{H}_d{d}", "masked_bwd", params, _mbwd(F32, wrap)))
for i in range(4):
    B, T, H, d = _shape(200)
    T = max(T, 2)
    T0 = int(_rng.integers(1, T))
    FUZZ.append((f"decode_f32_{i}_B{B}_T{T}_T0{T0}_H{H}_d{d}", "decode",
                 dict(B=B, T=T, H=H, d=d, T0=T0, es=0.7, seed=600 + i), _decode(F32)))
def _gemm_shape():
    """(B, T, D, H): D a multiple of 64 (the GEMMs' K), H dividing D with the
    generator width H * 3 floor(D / 3H) a multiple of 4 (the ABI's limits)."""
    while True:
        D = 64 * int(_rng.integers(1, 7))
        H = int(_rng.choice([h for h in (1, 2, 3, 4, 6, 8) if D % h == 0]))
        if (H * 3 * (D // H // 3)) % 4 == 0:
            return int(_rng.integers(1, 4)), int(_rng.integers(1, 301)), D, H


for i in range(5):
    B, T, D, H = _gemm_shape()
    FUZZ.append((f"gemm_{i}_B{B}_T{T}_D{D}_H{H}", "gemm",
                 dict(B=B, T=T, K=D, n_qkv=3 * D, n_gen=H * 3 * (D // H // 3), seed=700 + i), _gemm))
for i in range(3):
    B, T, D, H = _gemm_shape()
    FUZZ.append((f"edge_{i}_B{B}_T{T}_D{D}_H{H}", "edge", dict(B=B, T=T, K=D, H=H, seed=800 + i), _edge))
# longer sequences (one or two heads): more key tiles per query tile, the
# chained scan over more chunks
for i in range(4):
    T, H, d = int(_rng.integers(300, 2100)), int(_rng.integers(1, 3)), int(_rng.integers(3, 97))
    if i == 0:
        FUZZ.append((f"long_scan_attn_f16_T{T}_H{H}_d{d}", "scan_attn",
                     dict(B=1, T=T, H=H, d=d, io=BF16, op=F16, pf=S16, out=F32, es=0.3, seed=900 + i), _h16(F32)))
    elif i == 1:
        FUZZ.append((f"long_masked_causal_ring_bf16_T{T}_H{H}_d{d}", "masked",
                     dict(B=1, T=T, H=H, d=d, io=BF16, mode="causal", mask="ring", pf=S16, seed=900 + i),
                     _masked(BF16)))
    elif i == 2:
        FUZZ.append((f"long_bwd_f32_T{T}_H{H}_d{d}", "bwd", dict(B=1, T=T, H=H, d=d, es=0.5, seed=900 + i), _bwd(F32)))
    else:
        p = round(float(_rng.uniform(0.05, 0.5)), 3)
        FUZZ.append((f"long_dropout_inert_random_T{T}_H{H}_d{d}_p{p}", "masked_bwd",
                     dict(B=1, T=T, H=H, d=d, mode="inert", mask="random", io=F32, es=0.5, seed=900 + i,
                          drop={"p": p, "seed": 11, "offset": 2}), _drop(F32, False, p)))
for i in range(3):
    io = F32 if i % 2 == 0 else BF16
    e16 = 4 if io == F32 else 8                     # elements per 16 bytes: d a multiple of it
    n, dd = int(_rng.integers(1, 5000)), e16 * int(_rng.integers(1, 600))
    FUZZ.append((f"norm_{i}_io{io}_n{n}_d{dd}", "norm", dict(n=n, d=dd, io=io, seed=1000 + i), _norm(io)))
jobs.register("fuzz_shapes", [(name, params) for _, name, params, _ in FUZZ], timeout=1500)


@pytest.fixture(scope="module")
def fuzz_results():
    rc, out, res = jobs.result("fuzz_shapes")
    if rc != 0 or res is None:
        pytest.fail(f"emulated run failed (status {rc}):\n{out[-12000:]}")
    assert len(res["cases"]) == len(FUZZ)
    return {cid: r for (cid, *_), r in zip(FUZZ, res["cases"])}


@pytest.mark.emu_jobs("fuzz_shapes")
@pytest.mark.parametrize("cid", [c[0] for c in FUZZ])
def test_emulated_random_shapes(fuzz_results, cid):
    check = next(c[3] for c in FUZZ if c[0] == cid)
    r = fuzz_results[cid]
    assert r["stats"]["launches"] > 0
    check(r)
