"""Fingerprints of the gfx950 machine code of every kernel in a built
libholo_mi355x.so.

The library's .hip_fatbin section holds one offload bundle per compiled
source; each bundle's gfx950 code object is disassembled with ROCm's
llvm-objdump and every kernel's instruction stream (addresses and encoding
comments stripped; branch offsets are relative) is hashed. Two builds whose
fingerprints agree for a kernel run the same instructions for it. Used to
hold a rebuilt library to the kernels a GPU run validated or profiled
(tests/test_validated_kernels.py, bench.py's traffic figures). descriptors()
hashes each kernel's code-object metadata (register and LDS counts, the
argument layout), which the instruction stream leaves out.

    python -m holonomyawareattention_amd.kernel_code [library.so]   # {symbol: sha256}
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


CXXFILT = "/usr/bin/c++filt"       # binutils: names kernels as rocprofv3 prints them


def tools_present() -> bool:
    return all(os.path.exists(os.path.join(LLVM, t))
               for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump", "llvm-readobj"))


def _run(*cmd, stdin=None):
    r = subprocess.run(cmd, capture_output=True, text=True, input=stdin)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed: {r.stderr[-2000:]}")
    return r.stdout


def _code_objects(lib_path: str, tmp: str):
    """The gfx950 code objects of the library's offload bundles, unpacked
    into tmp (paths)."""
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
        if os.path.getsize(co) > 0:
            yield co


def fingerprints(lib_path: str) -> Dict[str, str]:
    """{kernel symbol: sha256 of its instruction stream} of every gfx950
    kernel in the library."""
    out: Dict[str, str] = {}
    with tempfile.TemporaryDirectory() as tmp:
        for co in _code_objects(lib_path, tmp):
            text = _run(os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", "--mcpu=gfx950", co)
            out.update(_per_symbol(text))
    return out


def descriptors(lib_path: str) -> Dict[str, str]:
    """{kernel symbol: sha256 of its code-object metadata} of every gfx950
    kernel: register counts (VGPR, AGPR, SGPR, spills), static LDS and
    scratch bytes, the kernel-argument layout and the workgroup limits -- what
    the instruction stream leaves out but the launch depends on (occupancy,
    argument offsets). The symbol names themselves are left out."""
    import yaml
    out: Dict[str, str] = {}
    with tempfile.TemporaryDirectory() as tmp:
        for co in _code_objects(lib_path, tmp):
            notes = _run(os.path.join(LLVM, "llvm-readobj"), "--notes", co)
            i0 = notes.index("---")
            i1 = notes.index("\n...", i0)
            for k in yaml.safe_load(notes[i0:i1])["amdhsa.kernels"]:
                d = {key: v for key, v in k.items() if key not in (".name", ".symbol", ".args")}
                d["args"] = [[a.get(".offset"), a.get(".size"), a.get(".value_kind")] for a in k.get(".args", [])]
                out[k[".name"]] = hashlib.sha256(json.dumps(d, sort_keys=True).encode()).hexdigest()
    return out


def demangle(symbols) -> Dict[str, str]:
    """{mangled: demangled} with binutils' c++filt, whose names are the ones
    rocprofv3 prints (both leave symbols with bf16 template arguments
    mangled). Identity where c++filt is absent."""
    symbols = list(symbols)
    if not os.path.exists(CXXFILT):
        return {n: n for n in symbols}
    out = _run(CXXFILT, stdin="\n".join(symbols) + "\n").splitlines()
    if len(out) != len(symbols):
        raise RuntimeError("c++filt returned a different number of names")
    return dict(zip(symbols, out))


def by_name(lib_path: str) -> Dict[str, str]:
    """fingerprints() keyed by both the mangled and the demangled symbol, so
    that a profiler's kernel name (either form) finds its kernel."""
    fp = fingerprints(lib_path)
    out = dict(fp)
    for mangled, plain in demangle(fp).items():
        out.setdefault(plain, fp[mangled])
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
    lib = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                             "libholo_mi355x.so")
    print(json.dumps(fingerprints(lib), indent=1, sort_keys=True))
