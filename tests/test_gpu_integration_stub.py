"""The documented Python binding (tests/integration/
attention_kernel_mi355x.py: ctypes on the library, torch for memory and the
stream) against the fp64 oracle. A stale signature in that file fails here.

Tolerances (written in the test): fp32 max-abs <= 2e-5; bf16 inputs with o in
fp32, max-abs <= 2e-3 against the oracle on the same bf16 q, k, v.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import holo_ref as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_side_binding(dtype):
    from tests.integration import attention_kernel_mi355x as stub
    B, T, H, d, es = 2, 200, 3, 48, 0.6
    m = 3 * (d // 3)
    g = torch.Generator(device=DEV).manual_seed(12)
    qkv = torch.randn(B, T, H, 3 * d, device=DEV, generator=g).to(dtype)
    gen = torch.randn(B, T, 2 * H * m, device=DEV, generator=g)
    q, k, v = qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:]
    gq, gk = gen[..., :H * m].view(B, T, H, m), gen[..., H * m:].view(B, T, H, m)
    o = stub.run_fwd_kernel_mi355x(q, k, v, gq, gk, es, 1.0 / math.sqrt(d),
                                   out_dtype=torch.float32 if dtype == torch.bfloat16 else None)
    torch.cuda.synchronize()
    f64 = lambda t: t.double().cpu().numpy().transpose(0, 2, 1, 3)
    a = es * (f64(gq) + np.roll(f64(gk), -1, axis=2))
    P, _ = R.geometry_blocks(a)
    ref = R.apply_blocks(P, R.causal_attention64(*(R.apply_blocks_T(P, f64(u)) for u in (q, k, v)),
                                                 1.0 / math.sqrt(d)))
    err = np.abs(f64(o) - ref).max()
    print(f"binding {dtype}: max-abs {err:.3e}")
    assert err <= (2e-5 if dtype == torch.float32 else 2e-3)
