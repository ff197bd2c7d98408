"""Decoder stack built from the path-ordered attention layer.

The reference's experiments wrap the attention module in a pre-LN block and
stack those blocks over a token embedding (experiments/session_cherry.py:286-294
for `HoloBlock`, :296-327 for the model and its `hidden`). This module keeps
that block and its parameter names, so its state_dict keys match the
reference's (`core.*`, `ln1.*`, `ln2.*`, `ff.0.*`, `ff.2.*`), and adds a
decoder with an LM head for the full-model benchmark.

The attention runs on the gfx950 kernels of `attention_kernel`; LayerNorm,
GELU and the MLP GEMMs are PyTorch operators (hipBLASLt GEMMs with fused bias).
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch
import torch.nn as nn

from .attention_kernel import PathOrderedGeometricMHA


class HoloBlock(nn.Module):
    """h + core(ln1(h)), then h + ff(ln2(h)), ff = Linear(d, 4d) -> GELU -> Linear(4d, d)
    (experiments/session_cherry.py:286-294)."""

    def __init__(self, d_model: int, n_heads: int, edge_scale: float, link_mode: str = "interaction"):
        super().__init__()
        self.core = PathOrderedGeometricMHA(d_model, n_heads=n_heads, edge_scale=edge_scale, mode="causal")
        self.core.link_mode = link_mode
        self.ln1, self.ln2 = nn.LayerNorm(d_model), nn.LayerNorm(d_model)
        self.ff = nn.Sequential(nn.Linear(d_model, 4 * d_model), nn.GELU(), nn.Linear(4 * d_model, d_model))

    def forward(self, h: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        h = h + self.core(self.ln1(h), attn_mask=mask, return_geometry=False)[0]
        return h + self.ff(self.ln2(h))


class HoloDecoder(nn.Module):
    """Token embedding, `n_layers` HoloBlocks and an LM head.

    `hidden(tokens)` is the reference model's `hidden` for its multi-layer holo
    arm (experiments/session_cherry.py:315-327): embed, then every block with
    the causal tril mask. `forward(tokens)` adds the LM head (no counterpart in
    the reference, whose experiments attach small task heads instead)."""

    def __init__(self, vocab: int, d_model: int, n_layers: int, n_heads: int, edge_scale: float,
                 link_mode: str = "interaction"):
        super().__init__()
        self.embed = nn.Embedding(vocab, d_model)
        self.blocks = nn.ModuleList([HoloBlock(d_model, n_heads, edge_scale, link_mode)
                                     for _ in range(n_layers)])
        self.lm_head = nn.Linear(d_model, vocab, bias=False)
        self._masks: Dict[Tuple[int, torch.device], torch.Tensor] = {}

    def causal_mask(self, L: int, device: torch.device) -> torch.Tensor:
        """tril(L) as a bool (L, L) tensor, built once per length and device
        (the attention layers check it once and then recognise it)."""
        key = (L, device)
        m = self._masks.get(key)
        if m is None:
            m = torch.ones(L, L, dtype=torch.bool, device=device).tril()
            self._masks[key] = m
        return m

    def hidden(self, tokens: torch.Tensor) -> torch.Tensor:
        h = self.embed(tokens)
        mask = self.causal_mask(h.shape[1], h.device)
        for b in self.blocks:
            h = b(h, mask)
        return h

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.hidden(tokens))
