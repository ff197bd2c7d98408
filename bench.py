"""Benchmark of the path-ordered attention forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2]

A step is one forward of the layer (x -> y: projections, link rotations and
prefix scan, transported causal attention, back-rotation, out-projection)
over one synthetic batch already resident in HBM. The default workload is
B=16, T=2048, H=16, d_head=96 (d_model=1536), bf16
activations, fp32 generator and rotation composition, edge_scale 0.05,
additive link generator, weights ~ N(0, 1/d_model), x ~ N(0, 1).

Prints one JSON line with the whole-job throughput (tokens/s), the layer's
TFLOP/s, per-stage HIP-event timings, the roofline of the attention core
(MFMA bf16) and of the scan stage (HBM), and a CPU baseline: the oracle's
step-by-step fp32 restatement of the reference chunked algorithm, timed on the
host cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "fwd tokens/s + TFLOP/s (B16 T2048 H16 d96 bf16), % of MFMA/HBM peak"
PEAK_BF16_TFLOPS = 2516.6          # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3           # MI355X fp32 MFMA
PEAK_HBM_GBS = 8000.0              # MI355X HBM3E

CONFIGS = {
    "cfg1": dict(B=8, T=128, D=192, H=4, dtype="fp32", es=0.05),
    "cfg2": dict(B=16, T=2048, D=1536, H=16, dtype="bf16", es=0.05),
    "cfg3": dict(B=2, T=32768, D=1536, H=16, dtype="bf16", es=0.05),
}


def scan_bytes_per_token_head(d: int, io_bytes: int, gen_bytes: int = 4, quat_bytes: int = 16,
                              gen_reads: int = 2) -> int:
    """Algorithmic HBM bytes of the scan stage per (token, head): read the
    generator output (gq and gk for the additive generator, one edge-MLP
    output for the interaction one: 3*nb fp32 each) and q, k, v (d each);
    write qh, kh, vh (d each) and P (nb quaternions: 16 B in fp32, 8 B as int16)."""
    nb = d // 3
    return gen_reads * 3 * nb * gen_bytes + 3 * d * io_bytes + 3 * d * io_bytes + nb * quat_bytes


def attention_core_flops(B, T, H, d) -> float:
    """QK^T and PV over the causal triangle: 2 * d * T(T+1) per (b, h)."""
    return 2.0 * d * T * (T + 1) * B * H


def projection_flops(B, T, D, m_total) -> float:
    """qkv (3D), generator (2 * H*m) and out (D) GEMMs."""
    return 2.0 * B * T * D * (3 * D + 2 * m_total + D)


def cpu_baseline(cfg, x_np, W, min_seconds=10.0, link_mode="additive"):
    """Oracle restatement of core/attention_fast_chunked.py (fp32, dense
    matrix_exp, sequential scan, BLOCK_K=64 streaming with the wrap branch),
    timed on whole batch rows of the workload (full T) until min_seconds have
    passed (at least one row)."""
    import torch
    from oracle import holo_ref
    B, T, H = x_np.shape[0], x_np.shape[1], cfg["H"]
    # the dense (T, d, d) prefix products of one row need T*H*d*d*4 bytes; past
    # 4096 tokens (config 3: 19 GB per row) a row's first 4096 tokens are timed
    Ts = min(T, 4096)
    Wt = {k: torch.as_tensor(v).float() for k, v in W.items()}
    rows = 0
    with torch.no_grad():
        holo_ref.forward_chunked(torch.as_tensor(x_np[:1, :64]).float(), Wt, H, cfg["es"], link_mode)  # warm-up
        t0 = time.perf_counter()
        while rows < B and (rows == 0 or time.perf_counter() - t0 < min_seconds):
            holo_ref.forward_chunked(torch.as_tensor(x_np[rows:rows + 1, :Ts]).float(), Wt, H, cfg["es"], link_mode)
            rows += 1
        dt = time.perf_counter() - t0
    span = f"full T={T} each" if Ts == T else (f"the first {Ts} of T={T} tokens each (a prefix: the "
                                               "attention cost per token grows with T, so the full "
                                               "sequence runs slower per token)")
    return {"value": rows * Ts / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "host_cpu_count": os.cpu_count(),
            "kind": "port", "seconds": round(dt, 3),
            "sample": f"batch rows 0..{rows - 1} of the same workload, {span} "
                      f"(H={H}, d_head={cfg['D'] // H}, fp32, the reference's dense SO(d) "
                      f"layout and chunked algorithm step by step, host threads={torch.get_num_threads()})"}


PMC_FETCH_SCALE = 2.0      # FETCH_SIZE reads 0.5x the bytes of a plain copy on this pool
PMC_WRITE_SCALE = 1.0      # WRITE_SIZE reads 1.0x


def pmc_summary(dirs):
    """Per-kernel mean FETCH_SIZE / WRITE_SIZE (KiB per dispatch, from
    rocprofv3 --pmc counter_collection.csv files under `dirs`), with the
    calibration factors measured on the --copy-probe copy (1 GiB read, 1 GiB
    written). Returns a dict keyed by kernel name."""
    import csv
    import glob
    acc = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = (r["Kernel_Name"], r["Counter_Name"])
                acc.setdefault(k, []).append(float(r["Counter_Value"]))
    copy = {c: max(v) for (n, c), v in acc.items() if "copyBuffer" in n}
    fs = (1 << 20) / copy["FETCH_SIZE"] if "FETCH_SIZE" in copy else PMC_FETCH_SCALE
    ws = (1 << 20) / copy["WRITE_SIZE"] if "WRITE_SIZE" in copy else PMC_WRITE_SCALE
    from holonomyawareattention_amd import build as holo_build
    # the build the counters were collected with: its sources digest, and
    # each kernel's instruction fingerprint (what traffic_from_profile matches)
    out = {"fetch_scale": fs, "write_scale": ws, "sources_sha": holo_build.library_digest(), "kernels": {}}
    code = library_code() or {}
    for (name, ctr), v in acc.items():
        if ctr not in ("FETCH_SIZE", "WRITE_SIZE"):
            continue
        e = out["kernels"].setdefault(name, {})
        scale = fs if ctr == "FETCH_SIZE" else ws
        e[ctr.lower() + "_bytes"] = sum(v) / len(v) * 1024 * scale
        e["dispatches"] = len(v)
        if name in code:
            e["code_sha256"] = code[name]
    return out


_LIB_CODE = {}


def library_code():
    """{kernel name (mangled and as profilers print it): instruction
    fingerprint} of the loaded library, computed once (None where ROCm's
    disassembler is absent)."""
    if "v" not in _LIB_CODE:
        from holonomyawareattention_amd import _lib, kernel_code
        try:
            _LIB_CODE["v"] = kernel_code.by_name(_lib.LIB_PATH) if kernel_code.tools_present() else None
        except Exception:          # the optional traffic field is then null; the bench line still prints
            _LIB_CODE["v"] = None
    return _LIB_CODE["v"]


def _base_name(name):
    """A profiler's kernel name without template arguments and parameters
    ("void holo::gemm_qkvg<256, ...>(holo::QkvgArgs)" -> "holo::gemm_qkvg");
    mangled names are returned as they are."""
    n = name.split("(")[0].split("<")[0]
    return n.split(" ")[-1]


def _same_code(code, name, sha):
    """True when the library's kernel `name` has instruction fingerprint
    `sha`, or, if no kernel has that name any more (a template parameter
    added with the old code as one of its values), when exactly one kernel of
    the same base name has it."""
    if name in code:
        return code[name] == sha
    hits = {n for n, h in code.items() if h == sha and _base_name(n) == _base_name(name) and "(" in n}
    return len(hits) == 1


def traffic_from_profile(config, kernel_prefix):
    """(HBM bytes per launch, source) of the kernels whose name contains any
    of `kernel_prefix` (summed), from the committed
    profiles/pmc_traffic_<config>.json. The bytes are not measured in this
    run: the profile records each kernel's instruction fingerprint in the
    build it was measured with (code_sha256), and the bytes are returned only
    when every matched kernel of the loaded library has the same fingerprint
    (the same machine code); otherwise None, so a profile of another kernel
    cannot pass for this one. `source` names the profile, the kernels and the
    outcome either way."""
    from holonomyawareattention_amd import build as holo_build
    rel = f"profiles/pmc_traffic_{config}.json"
    path = os.path.join(REPO, rel)
    lib_sha = holo_build.library_digest()
    if not os.path.exists(path):
        return None, {"profile": None, "library_sources_sha": lib_sha}
    data = json.load(open(path))
    matched = {name: e for name, e in data["kernels"].items()
               if any(p in name for p in kernel_prefix) and "fetch_size_bytes" in e and "write_size_bytes" in e}
    code = library_code()
    same = bool(matched) and code is not None and all(
        e.get("code_sha256") is not None and _same_code(code, name, e["code_sha256"]) for name, e in matched.items())
    src = {"profile": rel, "kernels": sorted(matched), "same_code": same,
           "measured_sources_sha": data.get("sources_sha"), "library_sources_sha": lib_sha,
           "measured_in_this_run": False}
    tot = sum(e["fetch_size_bytes"] + e["write_size_bytes"] for e in matched.values())
    return (tot if same else None), src


def orthogonality_report(m, x, config, kernels, torch):
    """Geometry at the longest prefix: P_{T-1} (and the holonomy) as the
    kernels apply them, i.e. the dense block rotations of the stored
    quaternions under the homogeneous map. Reports max |P^T P - I| entry,
    the induced infinity norm of P^T P - I (max absolute row sum, at most
    3x the entry max for 3x3 blocks) and the quaternion norm drift."""
    B, T, D = x.shape
    H = m.h
    d = D // H
    with torch.no_grad():
        q, k, v, gq, gk = m._link_inputs(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        qh, kh, vh_t, P, hol = kernels.geom_scan(q, k, v, gq, gk, m.edge_scale, want_hol=True)
        torch.cuda.synchronize()
        scan_ms = (time.perf_counter() - t0) * 1e3
        out = {"metric": "orthogonality of P at t = T-1", "config": {"workload": config, "B": B, "T": T, "H": H,
               "d_head": d, "edge_scale": m.edge_scale, "scan_chunk": 64}}
        for name, quat in (("P_last", P[:, :, T - 1].contiguous()), ("holonomy", hol)):
            R = kernels.quat_to_dense(quat, d).double()
            E = R.transpose(-1, -2) @ R - torch.eye(d, dtype=torch.float64, device=R.device)
            n2 = (quat.double() ** 2).sum(-1)
            out[name] = {"max_abs_entry": E.abs().max().item(),
                         "inf_norm": E.abs().sum(-1).max().item(),
                         "quat_norm2_drift": (n2 - 1).abs().max().item()}
        out["gate"] = "max_abs_entry <= 1e-4 (the entry maximum; the infinity norm is at most 3x it)"
        out["scan_ms_wall"] = scan_ms
    return out


DECODE_CFG = dict(B=64, T0=8192, D=1536, H=16, es=0.05)     # config 5


def decode_bench(args, torch, F, synth, kernels, Module):
    """Config 5: prefill 8192 tokens for 64 sequences, then time single-token
    decode steps (the module's decode_step, stage by stage with HIP events).
    The decode attention reads every cached key and value once per step:
    2 * B * H * (t + 1) * d * 2 bytes at position t, its roofline."""
    c = DECODE_CFG
    B, T0, D, H, es = c["B"], c["T0"], c["D"], c["H"], c["es"]
    d = D // H
    steps, warm = args.decode_steps, max(1, min(args.warmup, 8))
    dev, dt = torch.device("cuda:0"), torch.bfloat16
    inp = synth.layer_inputs(5, 1, 1, D, H, "additive")          # weights only (x is drawn below)
    m = Module(D, n_heads=H, edge_scale=es)
    m.link_mode = "additive"
    with torch.no_grad():
        for k, p in m.state_dict().items():
            if k in inp:
                p.copy_(torch.as_tensor(inp[k]))
    m = m.to(device=dev, dtype=dt).eval()
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(B, T0 + warm + steps, D, device=dev, generator=g).to(dt)
    t0 = time.perf_counter()
    _, st = m.prefill(x[:, :T0], capacity=T0 + warm + steps)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for i in range(warm):
        m.decode_step(x[:, T0 + i:T0 + i + 1], st)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    kv_bytes = 0
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    with torch.no_grad():
        for i in range(steps):
            pos = T0 + warm + i
            xt = x[:, pos:pos + 1]
            e = ev[i]
            e[0].record()
            q, k, v, gq, gk = m._link_inputs(xt)
            kernels.decode_geom(q[:, 0], k[:, 0], v[:, 0], st.g_prev, gk[:, 0], es, st.t, st.P, st.qh, st.kh, st.vh)
            st.g_prev = gq[:, 0].contiguous()
            e[1].record()
            o = kernels.decode_attention(st.qh, st.kh, st.vh, st.P, st.t, d, m.scale, workspace=st.workspace)
            e[2].record()
            F.linear(o.view(B, 1, D), m.out.weight)
            e[3].record()
            kv_bytes += 2 * B * H * (st.t + 1) * d * 2
            st.t += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    stage = [sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(steps)) for j in range(3)]
    attn_s = stage[1] * 1e-3
    ms = wall * 1e3 / steps
    # parity (untimed): every decoded row against the full-sequence forward of
    # the same tokens (row t of the causal forward depends on tokens 0..t only)
    n = warm + steps
    with torch.no_grad():
        L = T0 + n
        y_full = m(x[:, :L], torch.ones(L, L, dtype=torch.bool, device=dev).tril())[0][:, T0:]
        _, st2 = m.prefill(x[:, :T0], capacity=T0 + n)
        worst = 0.0
        for i in range(n):
            yt = m.decode_step(x[:, T0 + i:T0 + i + 1], st2)
            worst = max(worst, (yt[:, 0].float() - y_full[:, i].float()).abs().max().item())
    del y_full, st2
    return {"metric": "decode tokens/s (cfg5: B=64, prefix 8192, bf16), KV-read GB/s of the decode attention",
            "value": B * steps / wall, "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic (x ~ N(0,1) from torch.randn seeded 5; weights from the "
                                     "SplitMix64 generator, N(0,1/d_model))",
            "config": {"workload": "cfg5: incremental decode after a prefill", "global_batch": B, "prefix": T0,
                       "positions": [T0 + warm, T0 + warm + steps - 1], "n_heads": H, "d_head": d, "d_model": D,
                       "link_mode": "additive", "edge_scale": es, "parallelism": "single GPU"},
            "stages_ms_per_step": {"projections_and_geometry": stage[0] / steps, "decode_attention": stage[1] / steps,
                                   "out_projection": stage[2] / steps},
            "roofline": {"kernel": "decode_attn_split + decode_attn_combine (holo_decode_attn_fwd)", "bound": "hbm",
                         "achieved": kv_bytes / attn_s / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": kv_bytes / attn_s / 1e9 / PEAK_HBM_GBS, "traffic": None,
                         "bytes_per_step": kv_bytes / steps},
            "parity": {"max_abs_vs_full_forward": worst, "rows_checked": B * n,
                       "bound": "2e-2 (bf16: decode keeps the softmax weights in fp32, the full forward rounds "
                                "them to bf16 for its PV MFMA)"},
            "prefill_s": round(prefill_s, 3), "cpu_baseline": None}


def layer_mask(kind, T, torch, dev):
    """(mask or None, allowed pairs) of --mask: tril, none (every pair) or the
    ring mask of core/utils.py:59-75."""
    if kind == "tril":
        return torch.ones(T, T, dtype=torch.bool, device=dev).tril(), T * (T + 1) // 2
    if kind == "ring":
        i = torch.arange(T, device=dev)
        mask = torch.zeros(T, T, dtype=torch.bool, device=dev)
        for off in (-1, 0, 1):
            mask[i, (i + off) % T] = True
        return mask, int(mask.sum())
    return None, T * T


def train_bench(args, torch, F, synth, kernels, Module):
    """Forward + backward of one layer at a BASELINE config (default config 2)
    through the module's autograd path, and the backward timed alone on the
    saved forward state: the fused backward (holo_attn_bwd) for causal + tril,
    or with --exact-backward the exact path's (holo_attn_masked_bwd) for
    --mask none|ring or --mode inert; --dropout P (with --exact-backward, any
    mask) trains with attention dropout on the exact path's dropout pair
    (holo_attn_masked_dropout_fwd / _bwd), as the reference's kernel module
    sends such steps to its exact path. The backward attention's algorithmic
    work is 2.5x the forward's (recomputed QK^T, dP, dV, dK, dQ) over the
    pairs the mask allows."""
    cfg = CONFIGS[args.config]
    B, T, D, H, es = cfg["B"], cfg["T"], cfg["D"], cfg["H"], cfg["es"]
    d = D // H
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    dev = torch.device("cuda:0")
    inp = synth.layer_inputs(2, B, T, D, H, "additive")
    x = torch.as_tensor(inp.pop("x")).to(dev, dt)
    m = Module(D, n_heads=H, edge_scale=es, mode=args.mode, dropout=args.dropout)
    m.link_mode = "additive"
    m.exact_backward = args.exact_backward
    with torch.no_grad():
        for k, p in m.state_dict().items():
            if k in inp:
                p.copy_(torch.as_tensor(inp[k]))
    m = m.to(device=dev, dtype=dt).train()
    mask, pairs = layer_mask(args.mask, T, torch, dev)
    exact = args.exact_backward
    g = torch.Generator(device=dev).manual_seed(3)
    dy = torch.randn(B, T, D, device=dev, generator=g).to(dt)

    def step():
        m.zero_grad(set_to_none=True)
        y, _ = m(x, attn_mask=mask)
        y.backward(dy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the backward alone, on the state of one forward
    with torch.no_grad():
        q, k, v, gq, gk = m._link_inputs(x)
        do = torch.randn(B, T, H, d, device=dev, generator=g).to(dt)
        dqkv = torch.empty(B, T, H, 3 * d, dtype=dt, device=dev)
        dgq, dgk = torch.empty_like(gq), torch.empty_like(gk)
        lib = kernels._lib.load()
        dqs = (dqkv[..., :d], dqkv[..., d:2 * d], dqkv[..., 2 * d:])
        if exact:
            qh, kh, vh_t, P, hol = kernels.geom_scan(q, k, v, gq, gk, es, want_hol=args.mode == "causal",
                                                     p_format="f32", mode=args.mode)
            drop = dict(dropout_p=args.dropout, seed=0x5EED, offset=0)
            o, lse = kernels.attention_masked_train(qh, kh, vh_t, P, hol, d, m.scale, mode=args.mode, mask=mask,
                                                    **drop)
            ws = torch.empty(int(lib.holo_attn_masked_bwd_workspace_size(B, T, H, d, kernels._DT[dt],
                                                                          kernels._MODE[args.mode],
                                                                          int(mask is not None))),
                             dtype=torch.uint8, device=dev)
            run = lambda: kernels.attention_masked_backward(gq, gk, es, qh, kh, vh_t, P, hol, lse, o, do, d, m.scale,
                                                            *dqs, dgq, dgk, mode=args.mode, mask=mask, workspace=ws,
                                                            **drop)
        else:
            qh, kh, vh_t, P, _ = kernels.geom_scan(q, k, v, gq, gk, es, p_format="f32")
            lse = torch.empty((B, H, qh.shape[2]), dtype=torch.float32, device=dev)
            o = kernels.attention(qh, kh, vh_t, P, d, m.scale, lse=lse)
            ws = torch.empty(int(lib.holo_attn_bwd_workspace_size(B, T, H, d, kernels._DT[dt])),
                             dtype=torch.uint8, device=dev)
            run = lambda: kernels.attention_backward(gq, gk, es, qh, kh, vh_t, P, lse, o, do, d, m.scale,
                                                     *dqs, dgq, dgk, workspace=ws)
        for _ in range(3):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        bwd_ms = e0.elapsed_time(e1) / args.steps
    fl_bwd = 2.5 * 4 * d * pairs * B * H
    peak = PEAK_BF16_TFLOPS if dt == torch.bfloat16 else PEAK_FP32_TFLOPS
    ach = fl_bwd / (bwd_ms * 1e-3) / 1e12
    ms = wall * 1e3 / args.steps
    path = (f"{args.mode} mode, mask {args.mask}: exact path" if exact else "causal + tril")
    if args.dropout > 0:
        path += f", attention dropout p = {args.dropout}"
    kern = (("holo_attn_masked_dropout_bwd" if args.dropout > 0 else "holo_attn_masked_bwd")
            + " (bwd_prep + attn_bwd_masked_dkdv + attn_bwd_masked_dq"
            + (" + hol_torque" if args.mode == "causal" else "") + " + link_bwd)") if exact else \
        "holo_attn_bwd (bwd_prep + attn_bwd_dkdv + attn_bwd_dq + link_bwd)"
    return {"metric": f"training step tokens/s (forward + backward of one layer, {args.config})",
            "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": cfg["dtype"],
            "data": "synthetic (seeded SplitMix64/Box-Muller: x ~ N(0,1), weights ~ N(0,1/d_model); dy from "
                    "torch.randn seeded 3)",
            "config": {"workload": f"{args.config}: one layer forward + backward (all weight and input "
                                   f"gradients), {path}", "global_batch": B, "seq_len": T, "n_heads": H,
                       "d_head": d, "d_model": D, "link_mode": "additive", "edge_scale": es,
                       "mode": args.mode, "mask": args.mask, "dropout": args.dropout,
                       "parallelism": "single GPU"},
            "fused_backward_ms": bwd_ms,
            "roofline": {"kernel": kern, "bound": "mfma", "achieved": ach, "peak": peak, "unit": "TFLOP/s",
                         "frac": ach / peak, "traffic": None,
                         "work_per_launch": f"{fl_bwd:.4e} FLOP = 2.5 * 4*d*pairs*B*H ({pairs} allowed pairs "
                                            f"per (b, h))"},
            "cpu_baseline": None}


DECODER_CFG = dict(V=32000, D=1536, H=16, NL=12, B=8, T=4096, es=0.05)     # config 4


def decoder_bench(args, torch, F, kernels):
    """Config 4: forward of a random-init 12-layer pre-LN decoder (embedding,
    HoloBlocks, LM head) on uniform token ids, bf16. The attention layers record
    HIP events around their kernel stages inside the timed steps, which gives
    the attention kernel's share and roofline."""
    import numpy as np
    from holonomyawareattention_amd.decoder import HoloDecoder
    c = DECODER_CFG
    V, D, H, NL, B, T, es = c["V"], c["D"], c["H"], c["NL"], c["B"], c["T"], c["es"]
    d = D // H
    dev = torch.device("cuda:0")
    torch.manual_seed(4)                      # default nn init, on the device
    with torch.device(dev):
        m = HoloDecoder(V, D, NL, H, es, link_mode="additive")
    m = m.to(torch.bfloat16).eval()
    g = torch.Generator(device=dev).manual_seed(4)
    tok = torch.randint(0, V, (B, T), device=dev, generator=g)
    cores = [b.core for b in m.blocks]
    with torch.no_grad():
        y = m(tok)
        torch.cuda.synchronize()
        if not torch.isfinite(y.float()).all():
            raise RuntimeError("non-finite logits")
        del y
        for _ in range(args.warmup):
            m(tok)
        torch.cuda.synchronize()
        evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in cores]
               for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            for c_, e in zip(cores, evs[i]):
                c_._stage_events = e
            m(tok)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        for c_ in cores:
            c_._stage_events = None
    stage = np.zeros(4)
    for step in evs:
        for e in step:
            for j in range(4):
                stage[j] += e[j].elapsed_time(e[j + 1])
    stage_ms = stage / args.steps                     # summed over the 12 layers, per step
    ms = wall * 1e3 / args.steps
    m_total = H * m.blocks[0].core.m_dim
    fl_core = attention_core_flops(B, T, H, d)
    fl_layer = projection_flops(B, T, D, m_total) + fl_core + 2 * 2 * B * T * D * 4 * D
    fl_total = NL * fl_layer + 2 * B * T * D * V
    core_tflops = NL * fl_core / (stage_ms[2] * 1e-3) / 1e12
    out = {"metric": "decoder forward tokens/s (cfg4: 12 pre-LN layers, d_model 1536, H 16, vocab 32000, "
                     "B=8, T=4096, bf16)",
           "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (token ids uniform in [0, 32000) from torch.randint seeded 4; default nn "
                   "init seeded 4)",
           "config": {"workload": "cfg4: decoder forward to logits", "global_batch": B, "seq_len": T,
                      "n_layers": NL, "d_model": D, "n_heads": H, "d_head": d, "vocab": V,
                      "link_mode": "additive", "edge_scale": es, "parallelism": "single GPU"},
           "model_tflops": fl_total / (ms * 1e-3) / 1e12,
           "stages_ms_per_step": {"attention_layers_link_inputs": stage_ms[0], "attention_layers_scan": stage_ms[1],
                                  "attention_layers_attention_core": stage_ms[2],
                                  "attention_layers_out_projection": stage_ms[3],
                                  "rest (embedding, LayerNorms, MLPs, residuals, LM head)": ms - stage_ms.sum()},
           "roofline": {"kernel": "attn_fwd_h16 (holo_attn_fwd; fp16 operands), 12 launches per step", "bound": "mfma",
                        "achieved": core_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": core_tflops / PEAK_BF16_TFLOPS, "traffic": None,
                        "work_per_launch": f"{fl_core:.4e} FLOP = 2*d*T*(T+1)*B*H"}}
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = decoder_cpu_baseline(m, tok, c)
        except Exception as e:   # the GPU figure stands on its own
            out["cpu_baseline"] = {"error": repr(e)}
    else:
        out["cpu_baseline"] = None
    return out


def decoder_cpu_baseline(m, tok, c, Ts=512):
    """The same decoder on the host: the oracle's restatement of the reference
    chunked attention (fp32, dense matrix_exp, sequential scan) in every layer,
    torch fp32 LayerNorm / MLP / LM head, on batch row 0's first Ts tokens."""
    import torch
    from oracle import holo_ref
    H, es = c["H"], c["es"]
    f32 = lambda t: t.detach().float().cpu()
    with torch.no_grad():
        emb = f32(m.embed.weight)
        blocks = [(f32(b.ln1.weight), f32(b.ln1.bias), f32(b.ln2.weight), f32(b.ln2.bias),
                   {k: f32(v) for k, v in b.core.state_dict().items() if not k.startswith("edge_mlp")},
                   f32(b.ff[0].weight), f32(b.ff[0].bias), f32(b.ff[2].weight), f32(b.ff[2].bias))
                  for b in m.blocks]
        lm = f32(m.lm_head.weight)
        x = tok[:1, :Ts].cpu()
        t0 = time.perf_counter()
        h = emb[x]
        for l1w, l1b, l2w, l2b, Wc, w0, b0, w2, b2 in blocks:
            a = torch.nn.functional.layer_norm(h, (h.shape[-1],), l1w, l1b)
            h = h + holo_ref.forward_chunked(a, Wc, H, es)
            a = torch.nn.functional.layer_norm(h, (h.shape[-1],), l2w, l2b)
            h = h + torch.nn.functional.linear(torch.nn.functional.gelu(torch.nn.functional.linear(a, w0, b0)), w2, b2)
        h @ lm.T
        dt = time.perf_counter() - t0
    return {"value": Ts / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "host_cpu_count": os.cpu_count(), "kind": "port",
            "seconds": round(dt, 3),
            "sample": f"batch row 0, the first {Ts} of T={c['T']} tokens, all {c['NL']} layers and the LM "
                      f"head (fp32; attention = the reference's dense SO(d) layout and chunked algorithm step "
                      f"by step; host threads={torch.get_num_threads()}); a prefix, so per-token attention "
                      f"cost is lower than at the full T"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS) + ["cfg4"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with a plain 1 GiB device copy (PMC counter calibration)")
    ap.add_argument("--ortho", action="store_true",
                    help="config 3 geometry check: orthogonality of P at t = T-1 (one JSON line) and exit")
    ap.add_argument("--decode", action="store_true",
                    help="config 5: incremental decode after a prefill (one JSON line) and exit")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--link", default="additive", choices=["additive", "interaction"],
                    help="link generator of the layer (the reference module's default is interaction; the "
                         "configured workloads use the additive one)")
    ap.add_argument("--mask", default="tril", choices=["tril", "none", "ring"],
                    help="attention mask of the layer: tril (the configured workloads, the causal kernels) or, "
                         "on the exact-path kernels, none / the ring mask of core/utils.py:59-75")
    ap.add_argument("--mode", default="causal", choices=["causal", "inert"],
                    help="attention mode (inert runs the exact-path kernels with any mask)")
    ap.add_argument("--train", action="store_true",
                    help="forward + backward of one layer at --config (one JSON line) and exit")
    ap.add_argument("--fused-interaction", action="store_true",
                    help="with --link interaction: the edge MLP on the hand-written GEMM (the module's "
                         "fused_interaction option, off by default: run so far only on the CPU emulation)")
    ap.add_argument("--exact-backward", action="store_true",
                    help="with --train and --mask none|ring or --mode inert: the exact path's backward (the "
                         "module's exact_backward option, off by default: run so far only on the CPU emulation)")
    ap.add_argument("--dropout", type=float, default=0.0,
                    help="with --train and --exact-backward: attention dropout probability of the layer (the "
                         "exact path's dropout kernels, run so far only on the CPU emulation; any --mask)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc CSVs under DIR(s) as JSON and exit")
    args = ap.parse_args()
    if args.fused_interaction and args.link != "interaction":
        print("bench.py: --fused-interaction needs --link interaction", file=sys.stderr)
        sys.exit(2)
    if not (0.0 <= args.dropout < 1.0) or (args.dropout > 0 and not (args.train and args.exact_backward)):
        print("bench.py: --dropout takes 0 <= P < 1 and applies to --train with --exact-backward", file=sys.stderr)
        sys.exit(2)
    off_tril = args.mask != "tril" or args.mode != "causal" or args.dropout > 0
    if args.train and off_tril and not args.exact_backward:
        print("bench.py: --train with a mask other than tril or inert mode needs --exact-backward "
              "(without it the module's backward for these calls raises)", file=sys.stderr)
        sys.exit(2)
    if args.exact_backward and not (args.train and off_tril):
        print("bench.py: --exact-backward applies to --train with --mask none|ring, --mode inert or --dropout",
              file=sys.stderr)
        sys.exit(2)
    if args.pmc_summary:
        print(json.dumps(pmc_summary(args.pmc_summary), indent=1))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "the path shards over batch and heads with no communication in the forward, "
              "and this build runs and reports the single-GPU share.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import torch.nn.functional as F
    from holonomyawareattention_amd import kernels, synth
    from holonomyawareattention_amd.attention_kernel import PathOrderedGeometricMHA

    if args.decode:
        print(json.dumps(decode_bench(args, torch, F, synth, kernels, PathOrderedGeometricMHA)))
        return
    if args.config == "cfg4":
        print(json.dumps(decoder_bench(args, torch, F, kernels)))
        return
    if args.train:
        print(json.dumps(train_bench(args, torch, F, synth, kernels, PathOrderedGeometricMHA)))
        return
    cfg = CONFIGS[args.config]
    B, T, D, H, es = cfg["B"], cfg["T"], cfg["D"], cfg["H"], cfg["es"]
    d = D // H
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    dev = torch.device("cuda:0")

    inp = synth.layer_inputs(2, B, T, D, H, args.link)
    x_np = inp.pop("x")
    m = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=es, mode=args.mode)
    m.link_mode = args.link
    m.fused_interaction = args.fused_interaction
    with torch.no_grad():
        for k, p in m.state_dict().items():
            if k in inp:
                p.copy_(torch.as_tensor(inp[k]))
    m = m.to(device=dev, dtype=dt).eval()
    x = torch.as_tensor(x_np).to(device=dev, dtype=dt)
    if args.ortho:
        print(json.dumps(orthogonality_report(m, x, args.config, kernels, torch)))
        return
    mask, pairs = layer_mask(args.mask, T, torch, dev)
    exact = not m._tril_path(mask, T)

    pfmt = m._p_format(x, False)
    qbytes = 8 if pfmt == "snorm16" else 16

    with torch.no_grad():
        y_mod, _ = m(x, attn_mask=mask)
        torch.cuda.synchronize()
        if not torch.isfinite(y_mod.float()).all():
            raise RuntimeError("non-finite output")
        del y_mod
        for _ in range(args.warmup):
            m(x, attn_mask=mask)
        torch.cuda.synchronize()

        # whole-layer throughput through the public module; the module records
        # HIP events on its launch stream between its four stages, so the
        # per-stage (and roofline) timings come from these same timed launches
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            m._stage_events = evs[i]
            m(x, attn_mask=mask)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        m._stage_events = None
        if args.copy_probe:
            src = torch.ones(1 << 28, dtype=torch.float32, device=dev)     # 1 GiB
            dst = torch.empty_like(src)
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
    stage = np.zeros(4)
    for e in evs:
        for j in range(4):
            stage[j] += e[j].elapsed_time(e[j + 1])
    stage_ms = stage / args.steps
    ms_per_step = wall * 1e3 / args.steps
    tokens = B * T
    m_total = H * m.m_dim
    fl_core = 4.0 * d * pairs * B * H          # QK^T and PV over the allowed (i, j) pairs
    if args.link == "additive":
        fl_proj = projection_flops(B, T, D, m_total)
    else:                                   # qkv + out, and the edge MLP 2D -> 4D -> H*m
        fl_proj = 2.0 * B * T * D * 4 * D + 2.0 * B * T * (2 * D * 4 * D + 4 * D * m_total)
    io_bytes = 2 if dt == torch.bfloat16 else 4
    # generator bytes the scan reads per token-head: one fp32 row of g when the
    # fused projection GEMM formed g_t = gq(x_t) + gk(x_{t+1}) (or the edge MLP
    # wrote it), two (gq and gk) otherwise
    greads = 1 if (args.link != "additive" or m._fused_projection_ok(x)) else 2
    scan_bytes = scan_bytes_per_token_head(d, io_bytes, quat_bytes=qbytes, gen_reads=greads) * B * T * H
    core_peak = PEAK_BF16_TFLOPS if dt == torch.bfloat16 else PEAK_FP32_TFLOPS
    core_tflops = fl_core / (stage_ms[2] * 1e-3) / 1e12
    scan_gbs = scan_bytes / (stage_ms[1] * 1e-3) / 1e9
    # HBM traffic per launch from the committed counter profile of the same
    # machine code (None when a profiled kernel's fingerprint differs)
    no_profile = (None, {"profile": None, "reason": "no traffic profile for this workload"})
    attn_traffic = no_profile if exact else traffic_from_profile(
        args.config, ["attn_fwd_h16" if dt == torch.bfloat16 else "attn_fwdIf"])
    scan_traffic = (traffic_from_profile(args.config, ["scan_reset", "chunk_apply"]) if args.link == "additive"
                    else no_profile)

    out = {
        "metric": METRIC,
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded SplitMix64/Box-Muller: x ~ N(0,1), weights ~ N(0,1/d_model))",
        "config": {"workload": f"{args.config}: one path-ordered attention layer forward"
                               + (f" ({args.mode} mode, mask {args.mask}: exact-path kernels)" if exact else ""),
                   "global_batch": B, "seq_len": T, "n_heads": H, "d_head": d, "d_model": D,
                   "rotation": f"{d // 3} SO(3) blocks per head", "link_mode": args.link, "fused_interaction": args.fused_interaction,
                   "mode": args.mode, "mask": args.mask,
                   "attention_operands": ("bf16" if exact else "fp16") if dt == torch.bfloat16 else "fp32",
                   "edge_scale": es, "parallelism": "single GPU"},
        "layer_tflops": (fl_core + fl_proj) / (ms_per_step * 1e-3) / 1e12,
        "stages_ms": {"projections": stage_ms[0], "geom_scan": stage_ms[1],
                      "attention_core": stage_ms[2], "out_projection": stage_ms[3],
                      "sum": float(stage_ms.sum())},
        "roofline": {"kernel": ("attn_masked + wrap_queries + pack_mask (holo_attn_masked_fwd)" if exact
                                else ("attn_fwd_h16 (holo_attn_fwd; fp16 operands, fp32 accumulation)"
                                      if dt == torch.bfloat16 else "attn_fwd (holo_attn_fwd)")), "bound": "mfma",
                     "achieved": core_tflops, "peak": core_peak, "unit": "TFLOP/s",
                     "frac": core_tflops / core_peak,
                     "traffic": attn_traffic[0], "traffic_source": attn_traffic[1],
                     "work_per_launch": f"{fl_core:.4e} FLOP = 4*d*(allowed pairs {pairs})*B*H"},
        "roofline_scan": {"kernels": "scan_reset + chunk_apply (holo_geom_scan_fwd)",
                          "bound": "hbm", "achieved": scan_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": scan_gbs / PEAK_HBM_GBS,
                          "traffic": scan_traffic[0], "traffic_source": scan_traffic[1],
                          "bytes_per_launch": scan_bytes,
                          "bytes_per_token_head": scan_bytes_per_token_head(d, io_bytes, quat_bytes=qbytes,
                                                                            gen_reads=greads),
                          "p_format": pfmt},
    }
    if not args.no_cpu_baseline and not exact:
        W = {k: v for k, v in inp.items()}
        try:
            out["cpu_baseline"] = cpu_baseline(cfg, x_np, W, link_mode=args.link)
        except Exception as e:   # the GPU figure stands on its own
            out["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
