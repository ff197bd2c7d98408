"""Write the golden fixtures under tests/golden/ by running the reference.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden.py [/root/reference]

The reference's Python modules are imported by file path from the reference
tree and executed on the CPU. What the fixtures pin, that the mathematical
checks of the oracle cannot: the skew-vector index order and sign
(core/utils.py:20-26), the roll direction and pair order of the link generator
(core/attention_fast_chunked.py:74-75, :83-84), the head-major generator view
(:76), the left-multiplied prefix scan (:93), the P^T-in / P-out transport
sides (:108-110, :171), the finfo.min masking (:119, :146) and the per-head
interleaved q/k/v split (:69-71).

Inputs are regenerated from seeds by holonomyawareattention_amd.synth; the
tiny cases also store them. The SO(3)-block rotation model is fed to the
reference by scattering block generator rows into its dense layout.
Every file holds data only (inputs, expected outputs, checksums).
"""
from __future__ import annotations

import importlib.util
import os
import sys

sys.dont_write_bytecode = True      # write nothing into the read-only reference tree

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from holonomyawareattention_amd import synth  # noqa: E402
from oracle.holo_ref import dense_rows_from_block  # noqa: E402


def _load(ref_root: str, rel: str, name: str):
    core = os.path.join(ref_root, "core")
    if core not in sys.path:
        sys.path.insert(0, core)
    spec = importlib.util.spec_from_file_location(name, os.path.join(ref_root, rel))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _module(cls, D, H, es, link_mode, W, dtype):
    m = cls(D, n_heads=H, dropout=0.0, edge_scale=es, mode="causal").eval()
    m.link_mode = link_mode
    d = D // H
    sd = m.state_dict()
    new = {}
    for k, v in sd.items():
        if k in ("qkv.weight", "out.weight"):
            new[k] = torch.as_tensor(W[k])
        elif k in ("gqproj.weight", "gkproj.weight", "edge_mlp.2.weight", "edge_mlp.2.bias"):
            src = W.get(k)
            if src is None:
                new[k] = torch.zeros_like(v, dtype=torch.float64)
            else:
                new[k] = dense_rows_from_block(torch.as_tensor(src), H, d)
        elif k in W:
            new[k] = torch.as_tensor(W[k])
        else:
            new[k] = torch.zeros_like(v, dtype=torch.float64)
    m = m.to(dtype)
    m.load_state_dict({k: v.to(dtype) for k, v in new.items()})
    return m


def run_case(mod, name, seed, B, T, D, H, es, link_mode, dtype, store_inputs=True,
             y_rows=None, store_geometry=True):
    inp = synth.layer_inputs(seed, B, T, D, H, link_mode)
    x = inp.pop("x")
    m = _module(mod.PathOrderedGeometricMHA, D, H, es, link_mode, inp, dtype)
    xt = torch.as_tensor(x).to(dtype)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    with torch.no_grad():
        y, geom = m(xt, attn_mask=mask, return_geometry=True)
    out = dict(meta=np.array([seed, B, T, D, H], dtype=np.int64),
               edge_scale=np.array(es, dtype=np.float64),
               link_mode=np.array(link_mode), dtype=np.array(str(dtype)))
    if store_inputs:
        out["x"] = x
        for k, v in inp.items():
            out["w:" + k] = v
    else:
        out["x_checksum"] = np.array([x.sum(), np.abs(x).sum()])
        for k, v in inp.items():
            out["w_checksum:" + k] = np.array([v.sum(), np.abs(v).sum()])
    yn = y.double().numpy()
    if y_rows is None:
        out["y"] = yn
    else:
        out["y_rows"] = yn[:y_rows]
        out["y_row_sum"] = yn.sum(-1)
        out["y_row_abs"] = np.abs(yn).sum(-1)
    if store_geometry:
        out["P"] = geom["C"].double().numpy()
        out["Hol"] = geom["H"].double().numpy()
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}  |y|max={np.abs(yn).max():.3f}")


def run_original(mod, name, seed, B, T, D, H, es, link_mode):
    """core/attention.py (the O(L^3) arc-walk definition), fp64, tril mask."""
    inp = synth.layer_inputs(seed, B, T, D, H, link_mode)
    x = inp.pop("x")
    m = _module(mod.PathOrderedGeometricMHA, D, H, es, link_mode, inp, torch.float64)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    with torch.no_grad():
        y, geom = m(torch.as_tensor(x), attn_mask=mask, return_geometry=True)
    out = dict(meta=np.array([seed, B, T, D, H], dtype=np.int64),
               edge_scale=np.array(es, dtype=np.float64), link_mode=np.array(link_mode),
               x=x, y=y.numpy(), H=geom["H"].numpy(), C=geom["C"].numpy())
    for k, v in inp.items():
        out["w:" + k] = v
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


def main(ref_root: str):
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    chunked = _load(ref_root, "core/attention_fast_chunked.py", "_ref_chunked")
    original = _load(ref_root, "core/attention.py", "_ref_original")
    f64, f32 = torch.float64, torch.float32
    # tiny: d=12 (4 blocks), both generators, small and large angles
    run_case(chunked, "tiny_additive_es005_f64", 11, 2, 16, 48, 4, 0.05, "additive", f64)
    run_case(chunked, "tiny_additive_es15_f64", 12, 2, 16, 48, 4, 1.5, "additive", f64)
    run_case(chunked, "tiny_interaction_es15_f64", 13, 2, 16, 48, 4, 1.5, "interaction", f64)
    run_case(chunked, "tiny_additive_es15_f32", 12, 2, 16, 48, 4, 1.5, "additive", f32)
    # d=16: five blocks and one identity leftover dimension; T=70 crosses a key block
    run_case(chunked, "leftover_d16_es15_f64", 14, 1, 70, 32, 2, 1.5, "additive", f64)
    # BASELINE config 1 (B=8 T=128 D=192 H=4 d=48, fp32, edge_scale 0.05)
    run_case(chunked, "cfg1_additive_f32", 1, 8, 128, 192, 4, 0.05, "additive", f32,
             store_inputs=False, y_rows=2, store_geometry=False)
    run_case(chunked, "cfg1_additive_f64", 1, 8, 128, 192, 4, 0.05, "additive", f64,
             store_inputs=False, y_rows=2, store_geometry=False)
    # original arc-walk definition
    run_original(original, "original_arcwalk_es15_f64", 15, 2, 6, 24, 2, 1.5, "additive")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
