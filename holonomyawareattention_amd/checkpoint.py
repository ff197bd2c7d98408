"""Layout conversions between the reference's dense SO(d) generator and the
SO(3)-block generator of this package.

The reference's link generator emits, per head, the d(d-1)/2 entries of a
skew-symmetric d x d matrix in row-major upper-triangle order
(core/utils.py:20-26: entry (i, j), i < j, at index i*d - i(i+1)/2 + j-i-1).
This package's generator emits 3*(d//3) entries per head: block b's three are
the entries (3b, 3b+1), (3b, 3b+2), (3b+1, 3b+2) of that same matrix, every
other entry being zero. The functions here move generator weights between the
two layouts (gqproj.weight, gkproj.weight, edge_mlp.2.weight/bias: rows
H * m), so a reference checkpoint whose generator rows vanish outside the
blocks loads into PathOrderedGeometricMHA unchanged, and a block checkpoint
can be handed back to the reference's dense code.
"""
from __future__ import annotations

from typing import Dict, Mapping

import torch

# state_dict keys of the generator weights whose rows are per-head skew entries
GENERATOR_KEYS = ("gqproj.weight", "gkproj.weight", "edge_mlp.2.weight", "edge_mlp.2.bias")


def dense_width(d: int) -> int:
    """Generator entries per head in the reference's dense layout."""
    return d * (d - 1) // 2


def block_width(d: int) -> int:
    """Generator entries per head in the block layout (3 per SO(3) block)."""
    return 3 * (d // 3)


def block_positions(d: int) -> torch.Tensor:
    """Dense upper-triangle index of each block entry, (block_width(d),) int64:
    block b's entries (3b, 3b+1), (3b, 3b+2), (3b+1, 3b+2) in that order."""
    def tri(i: int, j: int) -> int:
        return i * d - i * (i + 1) // 2 + (j - i - 1)
    idx = []
    for b in range(d // 3):
        r = 3 * b
        idx += [tri(r, r + 1), tri(r, r + 2), tri(r + 1, r + 2)]
    return torch.tensor(idx, dtype=torch.int64)


def block_to_dense_rows(w: torch.Tensor, n_heads: int, d: int) -> torch.Tensor:
    """(H * block_width(d), ...) block-layout rows -> (H * dense_width(d), ...)
    dense-layout rows, zeros off the blocks."""
    mb, md = block_width(d), dense_width(d)
    if w.shape[0] != n_heads * mb:
        raise ValueError(f"expected {n_heads * mb} block rows, got {w.shape[0]}")
    hw = w.reshape(n_heads, mb, *w.shape[1:])
    out = w.new_zeros(n_heads, md, *w.shape[1:])
    out[:, block_positions(d).to(w.device)] = hw
    return out.reshape(n_heads * md, *w.shape[1:])


def dense_to_block_rows(w: torch.Tensor, n_heads: int, d: int, strict: bool = True) -> torch.Tensor:
    """(H * dense_width(d), ...) dense-layout rows -> (H * block_width(d), ...)
    block rows. With strict=True the rows off the blocks must be zero (then the
    conversion is exact); otherwise they are dropped (a projection onto the
    block model)."""
    mb, md = block_width(d), dense_width(d)
    if w.shape[0] != n_heads * md:
        raise ValueError(f"expected {n_heads * md} dense rows, got {w.shape[0]}")
    hw = w.reshape(n_heads, md, *w.shape[1:])
    pos = block_positions(d).to(w.device)
    if strict:
        off = torch.ones(md, dtype=torch.bool, device=w.device)
        off[pos] = False
        if bool((hw[:, off] != 0).any()):
            raise ValueError("dense generator rows are non-zero off the SO(3) blocks; the block model "
                             "cannot represent them (strict=False drops them)")
    return hw[:, pos].reshape(n_heads * mb, *w.shape[1:])


def from_reference_state_dict(sd: Mapping[str, torch.Tensor], n_heads: int, d_model: int,
                              strict: bool = True) -> Dict[str, torch.Tensor]:
    """A reference PathOrderedGeometricMHA state_dict (dense generator) in this
    package's layout: the generator keys converted, every other key kept."""
    d = d_model // n_heads
    out = dict(sd)
    for k in GENERATOR_KEYS:
        if k in out:
            out[k] = dense_to_block_rows(out[k], n_heads, d, strict)
    return out


def to_reference_state_dict(sd: Mapping[str, torch.Tensor], n_heads: int, d_model: int) -> Dict[str, torch.Tensor]:
    """This package's state_dict with the generator keys in the reference's
    dense layout."""
    d = d_model // n_heads
    out = dict(sd)
    for k in GENERATOR_KEYS:
        if k in out:
            out[k] = block_to_dense_rows(out[k], n_heads, d)
    return out


def skew_from_vec(v: torch.Tensor, d: int) -> torch.Tensor:
    """(..., m) generator entries -> (..., d, d) skew-symmetric matrices, for
    either layout: m = d(d-1)/2 is the reference's dense row-major upper
    triangle (core/utils.py:4-27), m = 3*(d//3) the block layout (block-diagonal
    result). The reference's rotation probe (experiments/session_state.py:
    278-279) can call this on a block model's generator output."""
    m = v.shape[-1]
    if m == block_width(d) and m != dense_width(d):
        pos = block_positions(d).to(v.device)
        v = v.new_zeros(*v.shape[:-1], dense_width(d)).index_copy(-1, pos, v)
    elif m != dense_width(d):
        raise ValueError(f"Expected last dim {dense_width(d)} (dense) or {block_width(d)} (blocks), got {m}")
    rows, cols = torch.triu_indices(d, d, offset=1, device=v.device)
    A = v.new_zeros(*v.shape[:-1], d, d)
    A[..., rows, cols] = v
    A[..., cols, rows] = -v
    return A
