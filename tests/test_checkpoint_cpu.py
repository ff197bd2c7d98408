"""The product's layout conversions (holonomyawareattention_amd.checkpoint)
against the oracle's block scatter and skew, which the golden fixtures written
from the reference pin (tests/test_oracle_golden.py)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import checkpoint as C
from holonomyawareattention_amd.attention_kernel import PathOrderedGeometricMHA
from oracle import holo_ref as R


@pytest.mark.parametrize("d", [3, 4, 12, 16, 48, 96])
def test_block_positions_match_oracle(d):
    assert C.block_positions(d).tolist() == R.block_to_dense_map(d).tolist()


@pytest.mark.parametrize("H,d", [(2, 12), (4, 16), (3, 48)])
def test_rows_round_trip(H, d):
    g = torch.Generator().manual_seed(d)
    w = torch.randn(H * C.block_width(d), 7, generator=g, dtype=torch.float64)
    dense = C.block_to_dense_rows(w, H, d)
    assert torch.equal(dense, R.dense_rows_from_block(w, H, d))
    assert torch.equal(C.dense_to_block_rows(dense, H, d), w)
    b = torch.randn(H * C.block_width(d), generator=g, dtype=torch.float64)       # a bias vector
    assert torch.equal(C.dense_to_block_rows(C.block_to_dense_rows(b, H, d), H, d), b)


def test_strict_rejects_off_block_rows():
    H, d = 2, 12
    dense = C.block_to_dense_rows(torch.randn(H * C.block_width(d), 5, dtype=torch.float64), H, d)
    dense[3] = 1.0                                        # (0, 4): between blocks 0 and 1
    with pytest.raises(ValueError):
        C.dense_to_block_rows(dense, H, d)
    kept = C.dense_to_block_rows(dense, H, d, strict=False)
    assert kept.shape == (H * C.block_width(d), 5)


@pytest.mark.parametrize("d", [6, 16, 48])
def test_skew_from_vec_both_layouts(d):
    g = torch.Generator().manual_seed(3)
    vd = torch.randn(5, C.dense_width(d), generator=g, dtype=torch.float64)
    assert torch.equal(C.skew_from_vec(vd, d), R.skew_from_vec(vd, d))
    vb = torch.randn(5, C.block_width(d), generator=g, dtype=torch.float64)
    scattered = R.dense_rows_from_block(vb.T, 1, d).T                  # (5, dense_width)
    assert torch.equal(C.skew_from_vec(vb, d), R.skew_from_vec(scattered, d))
    with pytest.raises(ValueError):
        C.skew_from_vec(torch.zeros(5, C.block_width(d) + 1, dtype=torch.float64), d)


@pytest.mark.parametrize("link_mode", ["additive", "interaction"])
def test_reference_state_dict_loads(link_mode):
    """A dense-layout state dict (the reference's generator shapes, rows zero
    off the blocks) converts and loads into the module, and converts back."""
    D, H = 48, 4
    d = D // H
    m = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=0.1)
    m.link_mode = link_mode
    ours = m.state_dict()
    dense = C.to_reference_state_dict(ours, H, D)
    assert dense["gqproj.weight"].shape == (H * C.dense_width(d), D)
    assert dense["edge_mlp.2.bias"].shape == (H * C.dense_width(d),)
    back = C.from_reference_state_dict(dense, H, D)
    m2 = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=0.1)
    m2.load_state_dict(back)
    for k, v in ours.items():
        assert torch.equal(m2.state_dict()[k], v), k
