"""The fused residual add + LayerNorm kernel (kernels.add_layernorm, the
decoder's norms outside autograd) against torch on the same inputs, and the
decoder's fused path against its torch path.

Tolerances (written in each test): h = x + delta is bit-identical to torch's
add in both dtypes (one rounding of an exact fp32 sum). fp32 y: max-abs
<= 2e-5 against torch's fp32 layer_norm of h (fp32 statistics in a different
summation order). bf16 y: within half a bf16 ulp (2^-8 relative) plus 1e-5
relative of the fp32 LayerNorm of the rounded h (one final rounding of a value
that agrees to fp32 accuracy).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from holonomyawareattention_amd import kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(n, d, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn(n, d, generator=g) * 2 + 0.5).to(DEV, dtype)
    dl = torch.randn(n, d, generator=g).to(DEV, dtype)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(DEV, dtype)
    b = (0.1 * torch.randn(d, generator=g)).to(DEV, dtype)
    return x, dl, w, b


@pytest.mark.parametrize("dtype,n,d", [(torch.float32, 1, 96), (torch.float32, 4097, 1536),
                                       (torch.float32, 37, 4096), (torch.float32, 5, 260),
                                       (torch.bfloat16, 4099, 1536), (torch.bfloat16, 3, 8192),
                                       (torch.bfloat16, 64, 520), (torch.bfloat16, 2, 96)])
def test_add_layernorm_matches_torch(dtype, n, d):
    print(f"add_layernorm {dtype} n={n} d={d}", flush=True)
    x, dl, w, b = _inputs(n, d, dtype, n + d)
    h, y = kernels.add_layernorm(x, dl, w, b, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(h, x + dl)
    ref = F.layer_norm(h.float(), (d,), w.float(), b.float(), 1e-5)
    err = (y.float() - ref).abs()
    if dtype == torch.float32:
        assert err.max().item() <= 2e-5, err.max().item()
    else:
        bound = (2.0 ** -8 + 1e-5) * ref.abs() + 1e-6
        assert bool((err <= bound).all()), (err - bound).max().item()


def test_add_layernorm_constant_row_and_batch_shape():
    """A constant row has zero variance: y = bias exactly (rstd = 1/sqrt(eps)
    times zero; d a power of two so the mean is exact); (B, T, d) inputs keep
    their shape."""
    d = 1024
    x = torch.full((2, 3, d), 1.25, device=DEV)
    dl = torch.full((2, 3, d), -0.5, device=DEV)
    w = torch.linspace(0.5, 1.5, d, device=DEV)
    b = torch.linspace(-1, 1, d, device=DEV)
    h, y = kernels.add_layernorm(x, dl, w, b, 1e-5)
    assert h.shape == y.shape == (2, 3, d)
    assert torch.equal(h, torch.full_like(h, 0.75))
    assert torch.equal(y, b.expand_as(y))


def test_decoder_fused_norms_match_torch_path():
    """hidden() outside autograd (fused add + LayerNorm) against the same model
    through torch's add and LayerNorm (autograd on), fp32: max-abs <= 1e-4
    relative to the largest hidden value (two layers; only the summation order
    of the norms' statistics differs)."""
    from holonomyawareattention_amd.decoder import HoloDecoder
    torch.manual_seed(0)
    m = HoloDecoder(40, 192, 2, 2, 0.3, "additive").to(DEV).eval()
    tok = torch.randint(0, 40, (2, 150), device=DEV)
    with torch.no_grad():
        h_fused = m.hidden(tok)
    h_torch = m.hidden(tok).detach()
    scale = h_torch.abs().max().item()
    err = (h_fused - h_torch).abs().max().item()
    print(f"decoder fused norms vs torch: max-abs {err:.3e} (max |h| {scale:.2f})")
    assert err <= 1e-4 * scale, err


def test_fused_norms_predicate_needs_matching_affine_norms():
    """The fused add + LayerNorm path is taken only for affine norms whose
    weights have the activations' dtype and device; otherwise the block runs
    torch's ops (no kernel launch in this test: the predicate alone)."""
    from holonomyawareattention_amd.decoder import HoloBlock, _fused_norms
    blk = HoloBlock(192, 2, 0.3, "additive").to(DEV, torch.bfloat16).eval()
    h = torch.zeros(1, 4, 192, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        assert _fused_norms(blk, h)
        blk.ln2.float()                                   # fp32 weights with bf16 activations
        assert not _fused_norms(blk, h)
        blk.ln2 = torch.nn.LayerNorm(192, elementwise_affine=False).to(DEV, torch.bfloat16)
        assert not _fused_norms(blk, h)
