"""The integration guide's code blocks are the committed files they claim to be.

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


def _top_level_args(text: str, open_at: int) -> tuple:
    """(argument count, end index) of the call whose '(' is at open_at."""
    depth, n, i, saw = 0, 0, open_at, False
    while i < len(text):
        ch = text[i]
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
            if depth == 0:
                return (n + 1 if saw else 0), i
        elif ch == "," and depth == 1:
            n += 1
        elif depth >= 1 and not ch.isspace():
            saw = True
        i += 1
    raise AssertionError("unbalanced call")


def test_every_c_snippet_call_has_the_header_arity():
    """Every holo_* call in the integration guide's C snippets (other than those
    eliding arguments with '...') passes as many arguments as the header's
    prototype declares, so a signature change that the page missed fails here."""
    hdr = open(os.path.join(REPO, "include", "holo_mi355x.h")).read()
    arity = {}
    for m in re.finditer(r"HOLO_API [^(]*?\b(holo_\w+)\(", hdr):
        n, end = _top_level_args(hdr, m.end() - 1)
        arity[m.group(1)] = 0 if hdr[m.end():end].strip() == "void" else n
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    checked = 0
    for block in re.finditer(r"```c\n(.*?)```", text, re.S):
        body = re.sub(r"/\*.*?\*/", " ", block.group(1), flags=re.S)
        for m in re.finditer(r"\b(holo_\w+)\(", body):
            name = m.group(1)
            if name not in arity:
                continue
            n, end = _top_level_args(body, m.end() - 1)
            if "..." in body[m.end():end]:
                continue
            assert n == arity[name], f"{name}: {n} arguments in INTEGRATION.md, {arity[name]} in the header"
            checked += 1
    assert checked >= 5
