"""Shape sweep through the drop-in module: head dimensions from 3 to the
supported maximum 96 (single blocks, leftover dims, the padded widths 32 / 64
/ 96, the scan's 16-byte-row path at 48 / 72 / 96), one to three heads and
sequence lengths around the 64-key tiles and 128-query workgroups, on the
causal + tril kernels and the exact path (no mask, causal; ring mask, inert),
against the float64 oracle.

Tolerance (written in the test): fp32 max-abs <= 2e-5 (the fp32 bar; the exact
path's wrap branch carries the holonomy) and NaN nowhere; bf16 max-abs
<= 2.5e-2 scaled as the other end-to-end tests scale it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import holo_ref as R
from tests._util import layer, make_module

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

HEAD_DIMS = [3, 5, 8, 24, 33, 64, 72, 94, 96]
SHAPES = [(1, 129, 1), (2, 70, 3), (2, 1, 2)]          # (B, T, H)
PATHS = [("causal", "tril"), ("causal", "none"), ("inert", "ring")]


@pytest.mark.parametrize("mode,mask_kind", PATHS)
@pytest.mark.parametrize("B,T,H", SHAPES)
@pytest.mark.parametrize("d", HEAD_DIMS)
def test_shape_sweep_fp32(d, B, T, H, mode, mask_kind):
    D = H * d
    print(f"shape sweep d={d} B={B} T={T} H={H} {mode}/{mask_kind}", flush=True)
    x, W = layer(90 + d, B, T, D, H, "additive", dtype=torch.float32)
    m = make_module(W, D, H, 0.7, "additive", torch.float32, DEV)
    m.mode = mode
    mask = {"tril": np.tril(np.ones((T, T), dtype=bool)), "none": None, "ring": R.ring_mask(T)}[mask_kind]
    mt = None if mask is None else torch.as_tensor(mask, device=DEV)
    with torch.no_grad():
        y, _ = m(torch.as_tensor(x, device=DEV, dtype=torch.float32), attn_mask=mt)
    torch.cuda.synchronize()
    y = y.double().cpu().numpy()
    ref = R.forward_exact_blocks(x, W, H, 0.7, mask=mask, mode=mode)
    assert np.isfinite(y).all()
    err = np.abs(y - ref).max()
    assert err <= 2e-5, err


@pytest.mark.parametrize("d", [5, 33, 72, 94])
def test_shape_sweep_bf16_tril(d):
    B, T, H = 2, 130, 2
    D = H * d
    x, W = layer(95 + d, B, T, D, H, "additive", dtype=torch.bfloat16)
    m = make_module(W, D, H, 0.7, "additive", torch.bfloat16, DEV)
    mask = torch.ones(T, T, dtype=torch.bool, device=DEV).tril()
    with torch.no_grad():
        y, _ = m(torch.as_tensor(x, device=DEV, dtype=torch.bfloat16), attn_mask=mask)
    torch.cuda.synchronize()
    y = y.double().cpu().numpy()
    ref = R.forward_blocks(x, W, H, 0.7)
    assert np.abs(y - ref).max() <= 2.5e-2 * max(1.0, np.abs(ref).max() / 4)


@pytest.mark.parametrize("T", [1, 64, 65, 257])
@pytest.mark.parametrize("d", [32, 64, 96])
def test_shape_sweep_bf16_tril_xcd_grid(d, T):
    """B*H = 8: the bf16 causal kernel's XCD-mapped grid of folded query-tile
    pairs (one fold at T <= 128, three at T = 257 with a ragged last tile),
    at each padded head width; same bar as the sweep above."""
    B, H = 2, 4
    D = H * d
    print(f"bf16 xcd grid d={d} T={T}", flush=True)
    x, W = layer(97 + d + T, B, T, D, H, "additive", dtype=torch.bfloat16)
    m = make_module(W, D, H, 0.7, "additive", torch.bfloat16, DEV)
    mask = torch.ones(T, T, dtype=torch.bool, device=DEV).tril()
    with torch.no_grad():
        y, _ = m(torch.as_tensor(x, device=DEV, dtype=torch.bfloat16), attn_mask=mask)
    torch.cuda.synchronize()
    y = y.double().cpu().numpy()
    ref = R.forward_blocks(x, W, H, 0.7)
    assert np.isfinite(y).all()
    assert np.abs(y - ref).max() <= 2.5e-2 * max(1.0, np.abs(ref).max() / 4)
