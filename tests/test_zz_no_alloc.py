"""holo_geom_scan_fwd_static (the scan with its chained state in the
library's static per-device array, no workspace) against holo_geom_scan_fwd
with a caller workspace: bit-identical outputs (the same kernels, a
deterministic scan) on calls in a row, each smaller than the one before, so a
later call runs on state a larger call left behind; inputs whose state exceeds
the array are rejected on the host before any launch."""
from __future__ import annotations

import pytest
import torch

from holonomyawareattention_amd import _lib, kernels
from tests._util import layer, make_module

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


def test_static_scratch_rejects_oversized_inputs():
    """Config 5's prefill (B=64, T=8192, H=16, d=96) needs 128 MiB of scan
    state: rejected with HOLO_ERR_UNSUPPORTED and a message, nothing launched."""
    lib = _lib.load()
    B, T, H, d = 64, 8192, 16, 96
    assert lib.holo_geom_scan_workspace_size(B, T, H, d) > _lib.HOLO_SCAN_STATIC_SCRATCH_BYTES
    rs, hs = H * 3 * d, 3 * d
    rc = lib.holo_geom_scan_fwd_static(B, T, H, d, _lib.HOLO_GEN_ADDITIVE, 0.05, _lib.HOLO_BF16, _lib.HOLO_F16,
                                       _lib.HOLO_F32, _lib.HOLO_QUAT_SNORM16, _lib.HOLO_MODE_CAUSAL,
                                       16, 2 * H * 96, 96, 16, 2 * H * 96, 96,
                                       16, rs, hs, 16, rs, hs, 16, rs, hs, 16, 16, 16, 16, None, None)
    assert rc == _lib.HOLO_ERR_UNSUPPORTED
    assert b"static scratch" in lib.holo_last_error()


@pytest.mark.gpu
def test_static_scratch_matches_workspace_scan():
    cases = [(16, 2048, 1536, 16, 0.05, torch.bfloat16, torch.float16, "snorm16"),    # config 2
             (3, 700, 384, 4, 0.6, torch.bfloat16, torch.bfloat16, "f32"),
             (2, 150, 96, 2, 0.9, torch.float32, torch.float32, "f32")]
    for B, T, D, H, es, dt, opdt, pf in cases:
        print(f"static scratch scan B={B} T={T} D={D} H={H} {dt} -> {opdt}", flush=True)
        x, W = layer(31, B, T, D, H, dtype=dt)
        m = make_module(W, D, H, es, "additive", dt, DEV)
        with torch.no_grad():
            q, k, v, gq, gk = m._link_inputs(torch.as_tensor(x).to(DEV, dt))
            ref = kernels.geom_scan(q, k, v, gq, gk, es, want_hol=True, p_format=pf, op_dtype=opdt)
            got = kernels.geom_scan(q, k, v, gq, gk, es, want_hol=True, p_format=pf, op_dtype=opdt,
                                    static_scratch=True)
            again = kernels.geom_scan(q, k, v, gq, gk, es, want_hol=True, p_format=pf, op_dtype=opdt,
                                      static_scratch=True)
        torch.cuda.synchronize()
        for a, b, c in zip(ref, got, again):
            assert torch.equal(a, b) and torch.equal(a, c)
