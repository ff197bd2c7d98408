"""Launch checker: every product kernel launched at the BASELINE configs'
full shapes (configs 1-5, and config 2's other generator, exact-path and
training workloads) on the CPU emulation of tests/emu, with every global
load and store, every buffer resource's range and every dynamic-LDS access
checked against allocations of exactly the documented sizes
(include/holo_mi355x.h). A violation aborts the child process with a report
naming the kernel source line, and the test fails with it.

The launches are the ABI calls the module makes (the same row and head
strides: the fused projection GEMM's q | k | v rows, the fp32 path's
concatenated GEMM output, interaction mode's broadcast bias row, the exact
path's bf16 operands and mask), on the same grids and LDS sizes as on the
GPU. Workgroups of independent launches (projection GEMM, attention, exact
path, LayerNorm, decode attention) are sampled -- the first and last ones of
the grid, which hold the largest offsets of the tile mappings -- because the
emulation runs each lane on the CPU; the chained scan, whose workgroups
depend on each other through its carries, always runs every workgroup.
Config 5's prefill scan runs at B = 2 (its launches at B = 64 differ only in
the batch offset, which config 2's B = 16 run and the B = 64 GEMM and
attention exercise); the exact-path and interaction layouts run at B = 4 of
config 2, the training step's backward at one batch row and two heads of
config 2's head size (also the exact path's training pair, off in the
module, with and without attention dropout). The fused interaction
generator's two GEMMs (off in the module) run
at config 2's shape with sampled workgroups.
"""
from __future__ import annotations

import os

import pytest

from tests.emu import build_emu, jobs

pytestmark = pytest.mark.skipif(not (os.path.exists(build_emu.CLANG) and os.path.exists(build_emu.ASAN_RT)),
                                reason="the CPU emulation needs ROCm's clang and its AddressSanitizer runtime")

CFG2 = dict(T=2048, D=1536, H=16)
S = [2, 2, 0]          # first two and last two workgroups of a sampled launch
CHECKS = [
    ("cfg1_fp32_layer", "layer_paths", dict(B=8, T=128, D=192, H=4, path="fp32")),
    ("cfg2_fused_bf16_layer", "layer", dict(B=16, **CFG2, sample_gemm=S, sample_attn=S, fill=False)),
    ("cfg2_interaction_layout", "layer_paths", dict(B=4, **CFG2, path="interaction", sample_attn=S)),
    ("cfg2_exact_no_mask_causal", "layer_paths", dict(B=4, **CFG2, path="exact", mask="none", sample_attn=S)),
    ("cfg2_exact_ring_inert", "layer_paths", dict(B=4, **CFG2, path="exact", mask="ring", mode="inert",
                                                  sample_attn=S)),
    ("cfg2_exact_random_causal", "layer_paths", dict(B=4, **CFG2, path="exact", mask="random", mode="causal",
                                                     sample_attn=S)),
    ("cfg2_train_backward_bf16", "bwd", dict(B=1, T=1024, H=2, d=96, io=1, es=0.05)),
    # the exact path's training pair (off in the module) at the same head
    # shape: causal mode with the ring mask (wrap pairs open), inert mode
    ("cfg2_exact_train_backward_ring_bf16", "masked_bwd", dict(B=1, T=1024, H=2, d=96, io=1, es=0.05,
                                                               mode="causal", mask="ring")),
    ("cfg2_exact_train_backward_inert_bf16", "masked_bwd", dict(B=1, T=1024, H=2, d=96, io=1, es=0.05,
                                                                mode="inert")),
    # the same pair with attention dropout (p = 0.1, the keep-mask kernel
    # too) under tril(T), the mask of a causal training step
    ("cfg2_dropout_train_backward_tril_bf16", "masked_bwd", dict(B=1, T=1024, H=2, d=96, io=1, es=0.05,
                                                                 mode="causal", mask="tril",
                                                                 drop={"p": 0.1, "seed": 2024, "offset": 1})),
    # the fused interaction generator (off in the module): first and last
    # four and every 997th workgroup of both GEMMs, written entries checked
    ("cfg2_fused_interaction_gemms", "edge", dict(B=16, T=2048, K=1536, H=16, sample=[4, 4, 997])),
    ("cfg3_layer", "layer", dict(B=2, T=32768, D=1536, H=16, sample_gemm=[1, 1, 0], sample_attn=[1, 1, 0],
                                 fill=False)),
    ("cfg4_layer", "layer", dict(B=8, T=4096, D=1536, H=16, sample_gemm=S, sample_attn=S, fill=False)),
    ("cfg4_add_layernorm", "norm", dict(n=8 * 4096, d=1536, io=1, sample=S)),
    ("cfg5_prefill_gemm_attention", "layer", dict(B=64, T=8192, D=1536, H=16, sample_gemm=S, sample_attn=[1, 1, 0],
                                                  fill=False, skip_scan=True)),
    ("cfg5_prefill_scan", "layer", dict(B=2, T=8192, D=1536, H=16, sample_gemm=[1, 1, 0], sample_attn=[1, 1, 0],
                                        fill=False)),
    ("cfg5_decode_first_and_last_step", "decode_bounds", dict(B=64, H=16, d=96, cap=8448, steps=[8192, 8447],
                                                              sample=[3, 3, 0])),
]


# four child processes of similar length, run at the same time
GROUPS = {"cfg1": 0, "cfg2": 1, "cfg3": 0, "cfg4": 2, "cfg5": 2}
N_GROUPS = 4


def _group(cid):
    if "interaction_gemms" in cid:
        return 3
    return 2 if "backward" in cid else GROUPS[cid.split("_")[0]]


for g in range(N_GROUPS):
    jobs.register(f"launch_checker_{g}", [(name, params) for cid, name, params in CHECKS if _group(cid) == g],
                  timeout=1800)


@pytest.fixture(scope="module")
def checked():
    out_all = {}
    for g in range(N_GROUPS):
        rc, out, res = jobs.result(f"launch_checker_{g}")
        if rc != 0 or res is None:
            pytest.fail(f"emulated launch check failed (status {rc}):\n{out[-12000:]}")
        ids = [cid for cid, *_ in CHECKS if _group(cid) == g]
        out_all.update(zip(ids, res["cases"]))
    return out_all


@pytest.mark.emu_jobs(*[f"launch_checker_{g}" for g in range(N_GROUPS)])
@pytest.mark.parametrize("cid", [c[0] for c in CHECKS])
def test_launch_in_bounds(checked, cid):
    r = checked[cid]
    st = r["stats"]
    assert st["launches"] > 0 and st["blocks"] > 0, r
    assert r.get("status", 0) == 0, r                      # no carry time-out, no fp16 overflow
    if cid == "cfg4_add_layernorm":
        assert r["h_err"] == 0.0 and r["y_err"] <= 2.0 ** -8 * r["y_max"] + 1e-5, r
    if cid == "cfg2_train_backward_bf16":
        assert all(v <= 3e-2 for k, v in r.items() if k.endswith("_fro")), r
    if cid.startswith("cfg2_exact_train_backward"):
        assert r["o_identical"] and all(v <= 3e-2 for k, v in r.items() if "_fro" in k), r
        assert (r["closing_edge_max"] > 1e-3) == ("ring" in cid), r
    if cid == "cfg2_dropout_train_backward_tril_bf16":
        assert r["keep_identical"] and r["o_drop_rel"] <= 2.5e-2, r
        assert all(v <= 3e-2 for k, v in r.items() if "_fro" in k), r
        assert r["closing_edge_max"] <= 1e-3, r
    if cid == "cfg2_fused_interaction_gemms":
        assert r["hid_err_over_bound"] <= 1.0 and r["qkv_err_over_bound"] <= 1.0 and r["g_err_over_bound"] <= 1.0, r
        assert r["written_hid"] > 0 and r["written_qkv"] > 0 and r["written_g"] > 0, r
    if cid.startswith("cfg5_decode"):
        assert all(v for k, v in r.items() if k.startswith("finite_")), r
