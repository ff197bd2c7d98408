"""The CPU oracle against the golden fixtures written by running the reference
(tests/golden/make_golden.py), plus planted mistakes that the fixtures catch."""
from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest
import torch

from oracle import holo_ref as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _case(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    seed, B, T, D, H = (int(v) for v in z["meta"])
    W = {k[2:]: z[k] for k in z.files if k.startswith("w:")}
    return z, B, T, D, H, float(z["edge_scale"]), str(z["link_mode"]), W


CHUNKED = ["tiny_additive_es005_f64", "tiny_additive_es15_f64", "tiny_interaction_es15_f64",
           "leftover_d16_es15_f64"]


@pytest.mark.parametrize("name", CHUNKED)
def test_chunked_restatement_matches_reference_fp64(name):
    z, B, T, D, H, es, lm, W = _case(name)
    Wt = {k: torch.as_tensor(v) for k, v in W.items()}
    y, g = R.forward_chunked(torch.as_tensor(z["x"]), Wt, H, es, lm, return_geometry=True)
    assert np.abs(y.numpy() - z["y"]).max() < 1e-12
    assert np.abs(g["C"].numpy() - z["P"]).max() < 1e-12
    assert np.abs(g["H"].numpy() - z["Hol"]).max() < 1e-12


def test_chunked_restatement_matches_reference_fp32_bitwise():
    """Same torch ops in the same order: the fp32 restatement reproduces the
    reference's fp32 run bit for bit."""
    z, B, T, D, H, es, lm, W = _case("tiny_additive_es15_f32")
    Wt = {k: torch.as_tensor(v).float() for k, v in W.items()}
    y, g = R.forward_chunked(torch.as_tensor(z["x"]).float(), Wt, H, es, lm, return_geometry=True)
    assert np.array_equal(y.double().numpy(), z["y"])
    assert np.array_equal(g["C"].double().numpy(), z["P"])


@pytest.mark.parametrize("name", CHUNKED)
def test_block_oracle_matches_reference(name):
    z, B, T, D, H, es, lm, W = _case(name)
    d = D // H
    y, parts = R.forward_blocks(z["x"], W, H, es, lm, return_parts=True)
    assert np.abs(y - z["y"]).max() < 1e-12
    assert np.abs(R.blocks_to_dense(parts["P"], d) - z["P"]).max() < 1e-12
    assert np.abs(R.blocks_to_dense(parts["Hol"], d) - z["Hol"]).max() < 1e-12


def test_arc_walk_matches_original_definition():
    z, B, T, D, H, es, lm, W = _case("original_arcwalk_es15_f64")
    y = R.forward_arc_walk(z["x"], W, H, es, lm)
    assert np.abs(y - z["y"]).max() < 1e-12
    # the original's C and H geometry are the block prefix products and holonomy
    d = D // H
    _, parts = R.forward_blocks(z["x"], W, H, es, lm, return_parts=True)
    assert np.abs(R.blocks_to_dense(parts["P"], d) - z["C"]).max() < 1e-12
    assert np.abs(R.blocks_to_dense(parts["Hol"], d) - z["H"]).max() < 1e-12


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_cfg1_reference_outputs(prec):
    """BASELINE config 1 regenerated from its seed: same inputs (checksums) and
    the oracle reproduces the reference's stored rows and row sums."""
    from tests._util import layer
    z = np.load(os.path.join(GOLDEN, f"cfg1_additive_{prec}.npz"))
    seed, B, T, D, H = (int(v) for v in z["meta"])
    dt = torch.float32 if prec == "f32" else torch.float64
    x, W = layer(seed, B, T, D, H, dtype=torch.float64)
    assert abs(x.sum() - z["x_checksum"][0]) < 1e-9 * z["x_checksum"][1]
    for k, v in W.items():
        cs = z["w_checksum:" + k]
        assert abs(v.sum() - cs[0]) <= 1e-9 * cs[1]
    Wt = {k: torch.as_tensor(v).to(dt) for k, v in W.items()}
    y = R.forward_chunked(torch.as_tensor(x).to(dt), Wt, H, 0.05).double().numpy()
    rows = z["y_rows"].shape[0]
    if prec == "f32":
        assert np.array_equal(y[:rows], z["y_rows"])
    else:
        assert np.abs(y[:rows] - z["y_rows"]).max() < 1e-12
    assert np.abs(y.sum(-1) - z["y_row_sum"]).max() < 1e-9 * D


# ---- planted mistakes: each must be caught by the fixtures ----
def _err_with(monkeypatch, name, patch):
    z, B, T, D, H, es, lm, W = _case(name)
    for target, fn in patch.items():
        monkeypatch.setattr(R, target, fn)
    y = R.forward_blocks(z["x"], W, H, es, lm)
    return np.abs(y - z["y"]).max()


def test_planted_skew_sign_is_caught(monkeypatch):
    orig = R.rodrigues
    err = _err_with(monkeypatch, "tiny_additive_es15_f64", {"rodrigues": lambda a: orig(-np.asarray(a))})
    assert err > 1e-3


def test_planted_transport_side_is_caught(monkeypatch):
    err = _err_with(monkeypatch, "tiny_additive_es15_f64",
                    {"apply_blocks_T": R.apply_blocks, "apply_blocks": R.apply_blocks_T})
    assert err > 1e-3


def test_planted_scan_order_is_caught(monkeypatch):
    def right_multiplied(G):
        *lead, Tm1, nb, _, _ = G.shape
        P = np.empty((*lead, Tm1 + 1, nb, 3, 3))
        cur = np.broadcast_to(np.eye(3), (*lead, nb, 3, 3)).copy()
        P[..., 0, :, :, :] = cur
        for t in range(Tm1):
            cur = cur @ G[..., t, :, :, :]
            P[..., t + 1, :, :, :] = cur
        return P
    err = _err_with(monkeypatch, "tiny_additive_es15_f64", {"prefix_blocks": right_multiplied})
    assert err > 1e-3


def test_planted_block_parameter_order_is_caught(monkeypatch):
    orig = R.rodrigues
    err = _err_with(monkeypatch, "tiny_additive_es15_f64",
                    {"rodrigues": lambda a: orig(np.asarray(a)[..., [1, 0, 2]])})
    assert err > 1e-3


def test_planted_generator_roll_direction_is_caught(monkeypatch):
    orig = R.generator_params

    def rolled_back(x, W, n_heads, edge_scale, link_mode):
        B, T, D = x.shape
        m = R.block_param_count(D // n_heads)
        gq = R._linear(x, W["gqproj.weight"]).view(B, T, n_heads, m).transpose(1, 2)
        gk = R._linear(x, W["gkproj.weight"]).view(B, T, n_heads, m).transpose(1, 2)
        return (gq + torch.roll(gk, shifts=1, dims=2)) * edge_scale
    err = _err_with(monkeypatch, "tiny_additive_es15_f64", {"generator_params": rolled_back})
    assert err > 1e-3
    assert orig is not rolled_back


def test_fixture_files_hold_data_only():
    for f in glob.glob(os.path.join(GOLDEN, "*.npz")):
        z = np.load(f, allow_pickle=False)          # raises on object arrays
        for k in z.files:
            assert z[k].dtype.kind in "fiub" or z[k].dtype.kind == "U", (f, k)
