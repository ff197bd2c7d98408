"""The fused backward (holo_attn_bwd through the module's autograd path) on
the GPU against the float64 backward oracle (oracle.holo_ref.backward_blocks,
pinned to torch autograd through the reference-step-by-step forward).

Tolerances (written in each test): fp32 max-abs <= 2e-5 relative to the
largest entry of each gradient (fp32 MFMA attention backward, fp32 suffix
sums); bf16 relative Frobenius <= 3e-2 against the oracle on the
bf16-rounded inputs (the attention products round q, k, v, do, the
probabilities and dS to bf16, as the forward's MFMAs do).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from holonomyawareattention_amd import kernels, synth
from oracle import holo_ref
from tests._util import layer, make_module, tril, round_to

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _grads(m, x, dy, dtype):
    xt = torch.as_tensor(x).to(DEV, dtype).requires_grad_(True)
    y, _ = m(xt, attn_mask=tril(x.shape[1], DEV))
    y.backward(torch.as_tensor(dy).to(DEV, dtype))
    torch.cuda.synchronize()
    out = {"x": xt.grad.double().cpu().numpy()}
    for k, p in m.named_parameters():
        if p.grad is not None:
            out[k] = p.grad.double().cpu().numpy()
    return out


@pytest.mark.parametrize("lm", ["additive", "interaction"])
@pytest.mark.parametrize("shape", [(2, 100, 96, 2, 0.9), (1, 130, 60, 4, 1.2), (2, 70, 64, 4, 0.5)])
def test_backward_fp32_matches_oracle(lm, shape):
    B, T, D, H, es = shape               # d = 48, 15 (Dp 32), 16 (one unrotated dim)
    x, W = layer(50, B, T, D, H, lm, dtype=torch.float32)
    dy = synth.normal(51, "dy", (B, T, D))
    m = make_module(W, D, H, es, lm, torch.float32, DEV)
    got = _grads(m, x, dy, torch.float32)
    ref = holo_ref.backward_blocks(x, W, H, es, dy, lm)
    worst = {}
    for k, v in got.items():
        r = ref[k]
        worst[k] = np.abs(v - r).max() / np.abs(r).max()
    print(lm, shape, {k: f"{e:.2e}" for k, e in worst.items()})
    assert set(worst) >= {"x", "qkv.weight", "out.weight"}
    for k, e in worst.items():
        assert e <= 2e-5, (k, e)


@pytest.mark.parametrize("lm", ["additive", "interaction"])
def test_backward_bf16_matches_oracle(lm):
    B, T, D, H, es = 2, 200, 192, 2, 0.3        # d = 96: the configured head size
    x, W = layer(52, B, T, D, H, lm, dtype=torch.bfloat16)
    dy = round_to(synth.normal(53, "dy", (B, T, D)), torch.bfloat16)
    m = make_module(W, D, H, es, lm, torch.bfloat16, DEV)
    got = _grads(m, x, dy, torch.bfloat16)
    ref = holo_ref.backward_blocks(x, W, H, es, dy, lm)
    rel = {k: np.linalg.norm(v - ref[k]) / np.linalg.norm(ref[k]) for k, v in got.items()}
    print(lm, {k: f"{e:.2e}" for k, e in rel.items()})
    for k, e in rel.items():
        assert e <= 3e-2, (k, e)


def test_kernel_level_gradients_fp32():
    """dq, dk, dv and the link gradient straight from kernels.attention_backward."""
    B, T, D, H, es = 2, 150, 96, 2, 1.0
    x, W = layer(54, B, T, D, H, "additive", dtype=torch.float32)
    dy = synth.normal(55, "dy", (B, T, D))
    ref = holo_ref.backward_blocks(x, W, H, es, dy)
    m = make_module(W, D, H, es, "additive", torch.float32, DEV)
    d, nb = D // H, D // H // 3
    with torch.no_grad():
        xt = torch.as_tensor(x).to(DEV, torch.float32)
        q, k, v, gq, gk = m._link_inputs(xt)
        qh, kh, vh_t, P, _ = kernels.geom_scan(q, k, v, gq, gk, es)
        lse = torch.empty((B, H, qh.shape[2]), dtype=torch.float32, device=DEV)
        o = kernels.attention(qh, kh, vh_t, P, d, m.scale, lse=lse)
        do = (torch.as_tensor(dy).to(DEV, torch.float32) @ m.out.weight).view(B, T, H, d)
        dq, dk, dv = (torch.empty(B, T, H, d, device=DEV) for _ in range(3))
        dgq, dgk = torch.empty_like(gq), torch.empty_like(gk)
        kernels.attention_backward(gq, gk, es, qh, kh, vh_t, P, lse, o, do, d, m.scale, dq, dk, dv, dgq, dgk)
        torch.cuda.synchronize()
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        r = ref[name].transpose(0, 2, 1, 3)          # (B,H,T,d) -> (B,T,H,d)
        err = np.abs(t.double().cpu().numpy() - r).max() / np.abs(r).max()
        assert err <= 2e-5, (name, err)
    da = ref["da"].transpose(0, 2, 1, 3)             # (B,T,H,m)
    got_dgq = dgq.double().cpu().numpy()
    assert np.abs(got_dgq - es * da).max() <= 2e-5 * np.abs(es * da).max()
    got_dgk = dgk.double().cpu().numpy()
    assert np.abs(got_dgk - np.roll(es * da, 1, axis=1)).max() <= 2e-5 * np.abs(es * da).max()


def test_backward_deterministic_bf16():
    """Two backward passes give bit-identical gradients (no atomics, fixed chain order)."""
    B, T, D, H, es = 2, 1000, 192, 2, 0.05
    x, W = layer(56, B, T, D, H, "additive", dtype=torch.bfloat16)
    dy = synth.normal(57, "dy", (B, T, D))
    m = make_module(W, D, H, es, "additive", torch.bfloat16, DEV)
    g1 = _grads(m, x, dy, torch.bfloat16)
    m.zero_grad(set_to_none=True)
    g2 = _grads(m, x, dy, torch.bfloat16)
    for k in g1:
        assert np.array_equal(g1[k], g2[k]), k
        assert np.isfinite(g1[k]).all(), k
