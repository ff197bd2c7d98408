"""The decoder stack (HoloDecoder: embedding, pre-LN HoloBlocks, LM head) on
the GPU against the float64 oracle (oracle.holo_ref.decoder_forward) on the
same weights and tokens.

Tolerances (written in each test): fp32 max-abs <= 2e-5 relative to the
largest logit (three layers of fp32 attention, LayerNorm and GEMMs; measured
1.3e-6 on MI355X); bf16
relative Frobenius <= 2e-2 against the oracle on the bf16-rounded weights
(every layer rounds its LayerNorm outputs, attention output, MLP activations
and the residual stream to bf16, each a ~4e-3 relative step).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import synth
from holonomyawareattention_amd.decoder import HoloDecoder
from oracle import holo_ref
from tests._util import round_to

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _model(W, V, D, NL, H, es, lm, dtype):
    m = HoloDecoder(V, D, NL, H, es, lm)
    sd = m.state_dict()
    with torch.no_grad():
        for k, v in W.items():
            sd[k].copy_(torch.as_tensor(v))
    return m.to(device=DEV, dtype=dtype).eval()


@pytest.mark.parametrize("dtype,lm", [(torch.float32, "additive"), (torch.float32, "interaction"),
                                      (torch.bfloat16, "additive")])
def test_decoder_matches_oracle(dtype, lm):
    V, D, H, NL, B, T, es = 50, 96, 2, 3, 2, 130, 0.5
    W = {k: round_to(v, dtype) for k, v in synth.decoder_inputs(7, V, D, H, NL, lm).items()}
    tok = synth.uniform_ints(7, "tokens", (B, T), V)
    m = _model(W, V, D, NL, H, es, lm, dtype)
    with torch.no_grad():
        logits = m(torch.as_tensor(tok, device=DEV)).double().cpu().numpy()
    ref = holo_ref.decoder_forward(tok, W, NL, H, es, lm)
    err = np.abs(logits - ref).max()
    rel = np.linalg.norm(logits - ref) / np.linalg.norm(ref)
    print(f"decoder {dtype} {lm}: max-abs {err:.3e} (max |logit| {np.abs(ref).max():.2f}), rel-F {rel:.3e}")
    if dtype == torch.float32:
        assert err <= 2e-5 * np.abs(ref).max(), err
    else:
        assert rel <= 2e-2, rel


def test_decoder_hidden_causal_prefix_bf16():
    """Hidden states of tokens 0..t are unchanged when later tokens change."""
    V, D, H, NL, B, T, es = 64, 96, 2, 2, 2, 200, 0.05
    W = synth.decoder_inputs(8, V, D, H, NL, "additive")
    m = _model(W, V, D, NL, H, es, "additive", torch.bfloat16)
    tok = torch.as_tensor(synth.uniform_ints(8, "tokens", (B, T), V), device=DEV)
    tok2 = tok.clone()
    tok2[:, 150:] = (tok2[:, 150:] + 1) % V
    with torch.no_grad():
        h1, h2 = m.hidden(tok), m.hidden(tok2)
    assert torch.equal(h1[:, :150], h2[:, :150])
    assert not torch.equal(h1[:, 150:], h2[:, 150:])
