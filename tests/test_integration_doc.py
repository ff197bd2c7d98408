"""INTEGRATION.md's code blocks are the committed files they claim to be.

A block preceded by `<!-- file: <path> -->` must equal that file byte for
byte; the files themselves are compiled (tests/c/integration_example.c, by
__graft_entry__.build()) or run on the GPU (tests/integration/
attention_kernel_mi355x.py, tests/test_gpu_integration_stub.py).
"""
from __future__ import annotations

import os
import re

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_BLOCK = re.compile(r"<!-- file: (?P<path>[^ ]+) -->\n```[a-z]*\n(?P<body>.*?)```", re.S)


def test_integration_blocks_are_the_committed_files():
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    blocks = list(_BLOCK.finditer(text))
    paths = {b.group("path") for b in blocks}
    assert paths == {"tests/integration/attention_kernel_mi355x.py", "tests/c/integration_example.c"}
    for b in blocks:
        with open(os.path.join(REPO, b.group("path"))) as f:
            assert f.read() == b.group("body"), b.group("path")


def test_c_example_matches_header_prototypes():
    """Every holo_* call in the C example names a function the header declares."""
    hdr = open(os.path.join(REPO, "include", "holo_mi355x.h")).read()
    declared = set(re.findall(r"HOLO_API [^(]*?\b(holo_\w+)\(", hdr))
    src = open(os.path.join(REPO, "tests", "c", "integration_example.c")).read()
    called = set(re.findall(r"\b(holo_\w+)\(", src)) - {"holo_example_core_bf16"}
    assert called and called <= declared, called - declared
