"""Build tests/emu/_build/libholo_emu.so: this package's HIP sources compiled
for x86-64 with AddressSanitizer against the CPU stand-in of the HIP runtime
(tests/emu/include/hip/hip_runtime.h), so that the kernels' own code runs on
the host lane by lane with every memory access bounds-checked. The library
exports the same C ABI as the gfx950 build (include/holo_mi355x.h) plus the
emu_* control functions of emu_runtime.cpp.

Test infrastructure only. The sources are used as they are except for three
mechanical substitutions, each asserted to match exactly as often as expected
(so a change in the product sources that they no longer fit fails the build):
  - `extern __shared__ __align__(16) unsigned char smem[];` (dynamic LDS)
    becomes a pointer to the launch's guarded LDS region;
  - the `s_waitcnt vmcnt(N)` inline assembly becomes emu::waitcnt_vm(N);
  - the ABI header's relative include path becomes a plain include.

    python tests/emu/build_emu.py
"""
from __future__ import annotations

import hashlib
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(REPO, "holonomyawareattention_amd", "csrc")
BUILD = os.path.join(HERE, "_build")
SRC_OUT = os.path.join(BUILD, "src")
LIB = os.path.join(BUILD, "libholo_emu.so")
STAMP = os.path.join(BUILD, "stamp.txt")

CLANG = "/opt/rocm/llvm/bin/clang++"
ASAN_RT = "/opt/rocm/llvm/lib/clang/22/lib/linux/libclang_rt.asan-x86_64.so"

FLAGS = ["-x", "c++", "-std=c++17", "-O1", "-g", "-fPIC", "-fno-omit-frame-pointer",
         "-fsanitize=address", "-fsanitize-address-use-after-return=never",
         # vector accesses need only dword alignment, as global memory under ROCm's
         # unaligned access mode on gfx9 (x86 would trap on 16-byte aligned moves)
         "-fmax-type-align=4",
         "-fvisibility=hidden", "-Wno-unknown-attributes", "-Wno-unused-result", "-Wno-ignored-attributes",
         "-I", os.path.join(HERE, "include"), "-I", HERE, "-I", os.path.join(REPO, "include"), "-I", SRC_OUT]

# (pattern, replacement, {file: expected count}); files not listed must not match
SUBSTITUTIONS = [
    (re.escape("extern __shared__ __align__(16) unsigned char smem[];"),
     "unsigned char* const smem = ::emu::dyn_lds();",
     {"holo_attn.hip": 2, "holo_gemm.hip": 1, "holo_attn_masked.hip": 1}),
    (re.escape('asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");'),
     "::emu::waitcnt_vm(N);",
     {"holo_attn_common.h": 1}),
    (re.escape('#include "../../include/holo_mi355x.h"'),
     '#include "holo_mi355x.h"',
     {"holo_abi.hip": 1}),
]


def _sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h")))


def _transform(name: str, text: str) -> str:
    for pat, rep, counts in SUBSTITUTIONS:
        text, n = re.subn(pat, rep, text)
        want = counts.get(name, 0)
        if want is None:           # any count (including none) is accepted for this file
            continue
        if n != want:
            raise RuntimeError(f"emu build: {name}: pattern {pat!r} matched {n} times, expected {want}")
    if re.search(r"\basm\s+volatile\s*\(\s*\"s_", text):
        raise RuntimeError(f"emu build: {name} holds GPU inline assembly the emulation does not model")
    return text


def _stamp() -> str:
    h = hashlib.sha256()
    for f in _sources():
        with open(os.path.join(CSRC, f), "rb") as fh:
            h.update(f.encode() + fh.read())
    for f in ("emu_device.h", "emu_runtime.cpp", "build_emu.py", os.path.join("include", "hip", "hip_runtime.h")):
        with open(os.path.join(HERE, f), "rb") as fh:
            h.update(f.encode() + fh.read())
    with open(os.path.join(REPO, "include", "holo_mi355x.h"), "rb") as fh:
        h.update(fh.read())
    return h.hexdigest()


def up_to_date() -> bool:
    if not os.path.exists(LIB) or not os.path.exists(STAMP):
        return False
    with open(STAMP) as fh:
        return fh.read().strip() == _stamp()


def build(force: bool = False, jobs: int = 8) -> str:
    """Compile (if the sources changed) and return the library's path."""
    if not force and up_to_date():
        return LIB
    if not os.path.exists(CLANG):
        raise RuntimeError(f"{CLANG} not found: the CPU emulation needs ROCm's clang")
    if os.path.exists(SRC_OUT):
        shutil.rmtree(SRC_OUT)
    os.makedirs(SRC_OUT)
    for f in _sources():
        with open(os.path.join(CSRC, f)) as fh:
            text = _transform(f, fh.read())
        with open(os.path.join(SRC_OUT, f), "w") as fh:
            fh.write(text)
    units = [os.path.join(SRC_OUT, f) for f in _sources() if f.endswith(".hip")]
    units.append(os.path.join(HERE, "emu_runtime.cpp"))

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        cmd = [CLANG, *FLAGS, "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"emu build failed on {os.path.basename(src)}:\n{r.stderr[-8000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, units))
    tmp = LIB + ".tmp"
    cmd = [CLANG, "-shared", "-fsanitize=address", "-shared-libasan", "-o", tmp, *objs, "-latomic"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"emu link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    with open(STAMP, "w") as fh:
        fh.write(_stamp())
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
