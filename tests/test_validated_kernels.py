"""Every kernel of the GPU-validated build compiles to the same gfx950
instructions in the library as built now (the fingerprints of
holonomyawareattention_amd/kernel_code.py against
tests/validated_kernels.json), with the same code-object metadata
(register, LDS and scratch counts, argument layout), so changes made without
a GPU run -- new kernels, new template modes -- provably leave the validated
kernels as they were. A kernel may change its symbol (e.g. a new template
parameter with the old behaviour as one value); it is matched by its
instructions and metadata. Kernels added since are listed, not checked."""
from __future__ import annotations

import json
import os

import pytest

from holonomyawareattention_amd import kernel_code

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "holonomyawareattention_amd", "libholo_mi355x.so")


@pytest.mark.skipif(not (os.path.exists(LIB) and kernel_code.tools_present()),
                    reason="library not built or ROCm's llvm tools absent")
def test_validated_kernels_unchanged():
    ref = json.load(open(os.path.join(REPO, "tests", "validated_kernels.json")))["kernels"]
    now = kernel_code.fingerprints(LIB)
    by_hash = {}
    for name, h in now.items():
        by_hash.setdefault(h, []).append(name)
    missing = [name for name, h in ref.items() if h not in by_hash]
    renamed = {name: by_hash[h] for name, h in ref.items() if h in by_hash and name not in by_hash[h]}
    added = sorted(set(now) - {n for h in ref.values() for n in by_hash.get(h, [])})
    print(f"{len(ref)} validated kernels, {len(renamed)} under a new symbol, {len(added)} added: {added}")
    assert not missing, f"validated kernels whose instructions changed: {missing}"
    desc_ref = json.load(open(os.path.join(REPO, "tests", "validated_kernels.json")))["descriptors"]
    desc_now = kernel_code.descriptors(LIB)
    assert set(desc_now) == set(now) and len(set(desc_now.values())) > len(now) // 4   # not a constant hash
    pairs = {(now[n], desc_now[n]) for n in now}
    changed = [name for name, h in ref.items() if (h, desc_ref[name]) not in pairs]
    assert not changed, f"validated kernels whose register, LDS or argument metadata changed: {changed}"
