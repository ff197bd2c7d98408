"""The decoder-stack oracle (oracle.holo_ref.decoder_forward) and the
decoder module's parameter layout, on the CPU.

Pin: with edge_scale = 0 every link rotation is the identity, so each block
is a standard pre-LN transformer block; torch's own nn.TransformerEncoderLayer
(norm_first, GELU, causal mask) with the same weights must give the same
logits in float64. A post-LN or misplaced residual, a tanh GELU, a wrong
LayerNorm epsilon or a mis-split qkv would each fail it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from holonomyawareattention_amd import synth
from oracle import holo_ref


def _encoder_stack(W, n_layers, D, H):
    d = D // H
    layers = []
    for i in range(n_layers):
        p = f"blocks.{i}."
        L = nn.TransformerEncoderLayer(D, H, dim_feedforward=4 * D, dropout=0.0, activation="gelu",
                                       batch_first=True, norm_first=True, layer_norm_eps=1e-5).double()
        wqkv = torch.as_tensor(W[p + "core.qkv.weight"]).view(H, 3, d, D)   # rows [q_h | k_h | v_h] per head
        with torch.no_grad():
            L.self_attn.in_proj_weight.copy_(wqkv.transpose(0, 1).reshape(3 * D, D))
            L.self_attn.in_proj_bias.zero_()
            L.self_attn.out_proj.weight.copy_(torch.as_tensor(W[p + "core.out.weight"]))
            L.self_attn.out_proj.bias.zero_()
            for ln, mod in (("ln1", L.norm1), ("ln2", L.norm2)):
                mod.weight.copy_(torch.as_tensor(W[p + ln + ".weight"]))
                mod.bias.copy_(torch.as_tensor(W[p + ln + ".bias"]))
            L.linear1.weight.copy_(torch.as_tensor(W[p + "ff.0.weight"]))
            L.linear1.bias.copy_(torch.as_tensor(W[p + "ff.0.bias"]))
            L.linear2.weight.copy_(torch.as_tensor(W[p + "ff.2.weight"]))
            L.linear2.bias.copy_(torch.as_tensor(W[p + "ff.2.bias"]))
        layers.append(L.eval())
    return layers


def test_flat_decoder_equals_torch_encoder_stack():
    V, D, H, NL, B, T = 37, 48, 4, 2, 2, 19
    W = synth.decoder_inputs(3, V, D, H, NL)
    tok = synth.uniform_ints(3, "tokens", (B, T), V)
    ref = holo_ref.decoder_forward(tok, W, NL, H, edge_scale=0.0)
    h = torch.as_tensor(W["embed.weight"])[torch.as_tensor(tok)]
    mask = nn.Transformer.generate_square_subsequent_mask(T, dtype=torch.float64)
    with torch.no_grad():
        for L in _encoder_stack(W, NL, D, H):
            h = L(h, src_mask=mask, is_causal=True)
        logits = (h @ torch.as_tensor(W["lm_head.weight"]).T).numpy()
    assert np.abs(logits - ref).max() <= 1e-10 * max(1.0, np.abs(ref).max())


def test_planted_post_ln_fails_the_pin():
    """A post-LN stack (residual added before the norm) is far from the oracle."""
    V, D, H, NL, B, T = 37, 48, 4, 2, 2, 11
    W = synth.decoder_inputs(4, V, D, H, NL)
    tok = synth.uniform_ints(4, "tokens", (B, T), V)
    ref = holo_ref.decoder_forward(tok, W, NL, H, edge_scale=0.0)
    h = torch.as_tensor(W["embed.weight"])[torch.as_tensor(tok)]
    mask = nn.Transformer.generate_square_subsequent_mask(T, dtype=torch.float64)
    with torch.no_grad():
        for L in _encoder_stack(W, NL, D, H):
            L.norm_first = False
            h = L(h, src_mask=mask, is_causal=True)
        logits = (h @ torch.as_tensor(W["lm_head.weight"]).T).numpy()
    assert np.abs(logits - ref).max() > 1e-2


@pytest.mark.parametrize("lm", ["additive", "interaction"])
def test_decoder_causal_prefix(lm):
    """Logits of tokens 0..t do not depend on later tokens (edge_scale > 0)."""
    V, D, H, NL, B, T = 29, 36, 2, 2, 1, 23
    W = synth.decoder_inputs(5, V, D, H, NL, lm)
    tok = synth.uniform_ints(5, "tokens", (B, T), V)
    full = holo_ref.decoder_forward(tok, W, NL, H, 0.7, lm)
    part = holo_ref.decoder_forward(tok[:, :15], W, NL, H, 0.7, lm)
    assert np.abs(full[:, :15] - part).max() <= 1e-10


@pytest.mark.parametrize("lm", ["additive", "interaction"])
def test_decoder_parameter_layout(lm):
    """Every generated weight is a parameter of HoloDecoder with the same shape;
    the only module parameters without one are the unused generator's."""
    from holonomyawareattention_amd.decoder import HoloDecoder
    V, D, H, NL = 31, 48, 4, 3
    W = synth.decoder_inputs(6, V, D, H, NL, lm)
    m = HoloDecoder(V, D, NL, H, 0.05, lm)
    sd = m.state_dict()
    for k, v in W.items():
        assert k in sd and tuple(sd[k].shape) == v.shape, k
    unused = "gqproj" if lm == "interaction" else "edge_mlp"
    for k in sd:
        if k not in W:
            assert f".core.{unused}" in k or (lm == "interaction" and ".core.gkproj" in k), k
    for b in m.blocks:
        assert b.core.link_mode == lm


def test_uniform_ints_range_and_determinism():
    a = synth.uniform_ints(9, "tokens", (4, 1000), 32000)
    b = synth.uniform_ints(9, "tokens", (4, 1000), 32000)
    assert a.dtype == np.int64 and (a == b).all()
    assert a.min() >= 0 and a.max() < 32000 and len(np.unique(a)) > 3500
