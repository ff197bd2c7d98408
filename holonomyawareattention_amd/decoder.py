"""Decoder stack built from the path-ordered attention layer.

The reference's experiments wrap the attention module in a pre-LN block and
stack those blocks over a token embedding (experiments/session_cherry.py:286-294
for `HoloBlock`, :296-327 for the model and its `hidden`). This module keeps
that block and its parameter names, so its state_dict keys match the
reference's (`core.*`, `ln1.*`, `ln2.*`, `ff.0.*`, `ff.2.*`), and adds a
decoder with an LM head for the full-model benchmark.

The attention runs on the gfx950 kernels of `attention_kernel`. Outside
autograd every residual add and the LayerNorm that follows it run as one
gfx950 kernel (`kernels.add_layernorm`); GELU and the MLP GEMMs are PyTorch
operators (hipBLASLt GEMMs with fused bias), and under autograd the norms and
adds are too (their gradients are torch's).
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
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
        if _fused_norms(self, h):
            return self.forward_fused(h, _ln(self.ln1, h), mask, None)[0]
        h = h + self.core(self.ln1(h), attn_mask=mask, return_geometry=False)[0]
        return h + self.ff(self.ln2(h))

    def forward_fused(self, h: torch.Tensor, a: torch.Tensor, mask: torch.Tensor,
                      next_ln: Optional[nn.LayerNorm]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """The block outside autograd, given a = ln1(h): each residual add runs
        fused with the LayerNorm after it (this block's ln2, then `next_ln`, the
        next block's ln1, when given). Returns (h_out, next_ln(h_out) or None)."""
        c = self.core(a, attn_mask=mask, return_geometry=False)[0]
        h, a = kernels.add_layernorm(h, c, self.ln2.weight, self.ln2.bias, self.ln2.eps)
        f = self.ff(a)
        if next_ln is None:
            return h + f, None
        return kernels.add_layernorm(h, f, next_ln.weight, next_ln.bias, next_ln.eps)


def _ln(ln: nn.LayerNorm, h: torch.Tensor) -> torch.Tensor:
    return F.layer_norm(h, ln.normalized_shape, ln.weight, ln.bias, ln.eps)


def _fused_norms(mod: nn.Module, h: torch.Tensor) -> bool:
    """The fused add + LayerNorm kernel serves calls outside autograd on the GPU
    (fp32 / bf16 rows whose width it supports); under autograd torch's
    differentiable ops run instead."""
    if not h.is_cuda or h.dtype not in (torch.float32, torch.bfloat16):
        return False
    if torch.is_grad_enabled() and (h.requires_grad or any(p.requires_grad for p in mod.parameters())):
        return False
    for ln in mod.modules():             # the kernel takes affine norms with weights of h's dtype and device
        if isinstance(ln, nn.LayerNorm) and (ln.weight is None or ln.bias is None or ln.weight.dtype != h.dtype
                                             or ln.bias.dtype != h.dtype or ln.weight.device != h.device):
            return False
    e16 = 16 // h.element_size()
    d = h.shape[-1]
    return d % e16 == 0 and d <= 1024 * e16


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
        if len(self.blocks) and _fused_norms(self, h):
            a = _ln(self.blocks[0].ln1, h)
            for i, b in enumerate(self.blocks):
                nxt = self.blocks[i + 1].ln1 if i + 1 < len(self.blocks) else None
                h, a = b.forward_fused(h, a, mask, nxt)
            return h
        for b in self.blocks:
            h = b(h, mask)
        return h

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.hidden(tokens))
