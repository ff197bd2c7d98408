"""Helpers shared by the tests: seeded layer inputs, module construction and
the bf16 rounding used to give the oracle exactly the values the GPU sees."""
from __future__ import annotations

import numpy as np
import torch

from holonomyawareattention_amd import synth


def round_to(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """float64 copy of `a` after rounding to `dtype` (identity for float64)."""
    return torch.as_tensor(np.asarray(a)).to(dtype).double().numpy()


def layer(seed, B, T, D, H, link_mode="additive", dtype=torch.float32):
    """Seeded inputs rounded to `dtype`: returns (x, W) as float64 numpy."""
    inp = synth.layer_inputs(seed, B, T, D, H, link_mode)
    x = round_to(inp.pop("x"), dtype)
    W = {k: round_to(v, dtype) for k, v in inp.items()}
    return x, W


def make_module(W, D, H, es, link_mode, dtype, device):
    from holonomyawareattention_amd.attention_kernel import PathOrderedGeometricMHA
    m = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=es)
    m.link_mode = link_mode
    sd = m.state_dict()
    with torch.no_grad():
        for k in sd:
            if k in W:
                sd[k].copy_(torch.as_tensor(W[k]))
    return m.to(device=device, dtype=dtype).eval()


def tril(T, device):
    return torch.ones(T, T, dtype=torch.bool, device=device).tril()


def run_module(m, x, device, dtype, return_geometry=False):
    xt = torch.as_tensor(x).to(device=device, dtype=dtype)
    with torch.no_grad():
        y, g = m(xt, attn_mask=tril(x.shape[1], device), return_geometry=return_geometry)
    torch.cuda.synchronize()
    return y, g
