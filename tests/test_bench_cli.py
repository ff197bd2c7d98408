"""bench.py refuses more than one GPU with a message (nothing is launched)."""
from __future__ import annotations

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_traffic_is_reported_only_for_the_profiled_build(monkeypatch):
    """roofline.traffic comes from the committed counter profile only when the
    profile's sources digest equals the loaded library's build stamp; a
    different or missing stamp gives None, and the line names the profile and
    both digests either way."""
    sys.path.insert(0, REPO)
    import bench
    from holonomyawareattention_amd import build
    prof = bench.json.load(open(os.path.join(REPO, "profiles", "pmc_traffic_cfg2.json")))
    sha = prof["sources_sha"]
    monkeypatch.setattr(build, "library_digest", lambda: sha)
    t, src = bench.traffic_from_profile("cfg2", ["scan_reset", "chunk_apply"])
    assert t is not None and t > 9e8 and src["same_build"] and src["profile"] == "profiles/pmc_traffic_cfg2.json"
    assert not src["measured_in_this_run"]
    monkeypatch.setattr(build, "library_digest", lambda: "0" * 64)
    t, src = bench.traffic_from_profile("cfg2", ["scan_reset", "chunk_apply"])
    assert t is None and not src["same_build"] and src["measured_sources_sha"] == sha
    monkeypatch.setattr(build, "library_digest", lambda: None)
    assert bench.traffic_from_profile("cfg2", ["attn_fwd_h16"])[0] is None
    assert bench.traffic_from_profile("cfg9", ["attn_fwd_h16"]) == (None, {"profile": None, "library_sources_sha": None})


def test_library_stamp_is_the_sources_digest():
    """build() writes the digest of what it compiled next to the library (a
    source edit without a rebuild leaves the old stamp, so a stale library
    is not matched to a new profile either)."""
    from holonomyawareattention_amd import build
    if not (os.path.exists(build.LIB_PATH) and os.path.exists(build.STAMP_PATH)):
        import pytest
        pytest.skip("library not built")
    assert build.library_digest() == build.sources_digest()
