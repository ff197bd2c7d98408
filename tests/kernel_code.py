"""Fingerprints of the gfx950 machine code of every kernel in a built
libholo_mi355x.so (test infrastructure only).

The library's .hip_fatbin section holds one offload bundle per compiled
source; each bundle's gfx950 code object is disassembled with ROCm's
llvm-objdump and every kernel's instruction stream (addresses and encoding
comments stripped; branch offsets are relative) is hashed. Two builds whose
fingerprints agree for a kernel run the same instructions for it.

    python -m tests.kernel_code [library.so]      # prints {symbol: sha256}
"""
from __future__ import annotations

import hashlib
import json
import os
import re
import subprocess
import sys
import tempfile
from typing import Dict

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def tools_present() -> bool:
    return all(os.path.exists(os.path.join(LLVM, t)) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


def _run(*cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed: {r.stderr[-2000:]}")
    return r.stdout


def fingerprints(lib_path: str) -> Dict[str, str]:
    """{kernel symbol: sha256 of its instruction stream} of every gfx950
    kernel in the library."""
    out: Dict[str, str] = {}
    with tempfile.TemporaryDirectory() as tmp:
        fat = os.path.join(tmp, "fatbin")
        _run(os.path.join(LLVM, "llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", lib_path,
             os.path.join(tmp, "discard.so"))
        data = open(fat, "rb").read()
        starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
        for n, s in enumerate(starts):
            e = starts[n + 1] if n + 1 < len(starts) else len(data)
            bun = os.path.join(tmp, f"b{n}")
            with open(bun, "wb") as fh:
                fh.write(data[s:e])
            co = os.path.join(tmp, f"co{n}")
            _run(os.path.join(LLVM, "clang-offload-bundler"), "--type=o", f"--targets={TARGET}",
                 f"--input={bun}", f"--output={co}", "--unbundle")
            if os.path.getsize(co) == 0:
                continue
            text = _run(os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", "--mcpu=gfx950", co)
            out.update(_per_symbol(text))
    return out


def _per_symbol(text: str) -> Dict[str, str]:
    res: Dict[str, str] = {}
    name, lines = None, []

    def close():
        if name is not None and lines:
            res[name] = hashlib.sha256("\n".join(lines).encode()).hexdigest()

    for raw in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", raw)
        if m:
            close()
            name, lines = m.group(1), []
            continue
        if name is None:
            continue
        t = raw.split("//")[0].strip()
        if t and not t.startswith(("Disassembly of", ".")):
            lines.append(re.sub(r"\s+", " ", t))
    close()
    return {k: v for k, v in res.items() if not k.endswith(".kd")}


if __name__ == "__main__":
    lib = sys.argv[1] if len(sys.argv) > 1 else os.path.join(
        os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "holonomyawareattention_amd", "libholo_mi355x.so")
    print(json.dumps(fingerprints(lib), indent=1, sort_keys=True))
