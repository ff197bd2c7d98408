"""Build libholo_mi355x.so (gfx950) in-tree with hipcc.

    python -m holonomyawareattention_amd.build

Every HIP source under csrc/ is compiled for gfx950 only, with packed-fp32
instruction selection disabled, and linked into one shared library next to
this file. The library exports exactly the C ABI of include/holo_mi355x.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB_NAME = "libholo_mi355x.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
SOURCES = ["holo_abi.hip", "holo_scan.hip", "holo_attn.hip", "holo_decode.hip", "holo_bwd.hip", "holo_norm.hip",
           "holo_attn_masked.hip", "holo_gemm.hip", "holo_bwd_masked.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wno-unused-result",
    "-I", os.path.join(REPO, "include"),
]


STAMP_PATH = LIB_PATH + ".sources"


def sources_digest() -> str:
    """sha256 of what the library is compiled from: the compiler flags, every
    HIP source and header under csrc/ and the ABI header. build_library()
    writes it next to the library, so a measurement recorded with one build
    (e.g. an HBM-traffic profile) can be matched against the library loaded
    later."""
    import hashlib
    h = hashlib.sha256(" ".join(HIPCC_FLAGS[:-2]).encode())
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(CSRC, name), "rb") as fh:
                h.update(name.encode() + b"\0" + fh.read())
    with open(os.path.join(REPO, "include", "holo_mi355x.h"), "rb") as fh:
        h.update(fh.read())
    return h.hexdigest()


def library_digest():
    """The sources digest recorded when the present library was built, or None."""
    try:
        with open(STAMP_PATH) as fh:
            return fh.read().strip() or None
    except OSError:
        return None


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 HIP library cannot be built")


def build_library(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        cmd = [hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
        if verbose and r.stderr.strip():
            print(r.stderr[-2000:], file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB_PATH)
    with open(STAMP_PATH, "w") as fh:
        fh.write(sources_digest() + "\n")
    return LIB_PATH


C_SMOKE_SRC = os.path.join(REPO, "tests", "c", "abi_smoke.c")
C_EXAMPLE_SRC = os.path.join(REPO, "tests", "c", "integration_example.c")
C_TRAIN_EXAMPLE_SRC = os.path.join(REPO, "tests", "c", "exact_train_example.c")
C_SMOKE_BIN = os.path.join(PKG, "_build", "abi_smoke")


def build_c_smoke() -> str:
    """Compile the C caller of the ABI (tests/c/abi_smoke.c, which also calls
    the documented C binding example, tests/c/integration_example.c, and
    links the exact path's training example, tests/c/exact_train_example.c)
    with gcc against the HIP runtime and this library (no PyTorch); returns
    the binary's path. A stale signature in any of them fails here."""
    os.makedirs(os.path.dirname(C_SMOKE_BIN), exist_ok=True)
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler found for the ABI smoke driver")
    cmd = [cc, "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I/opt/rocm/include", "-I", os.path.join(REPO, "include"), C_SMOKE_SRC, C_EXAMPLE_SRC,
           C_TRAIN_EXAMPLE_SRC, "-o", C_SMOKE_BIN,
           "-L", PKG, "-lholo_mi355x", "-L/opt/rocm/lib", "-lamdhip64", "-lm", "-Wl,-rpath," + PKG,
           "-Wl,-rpath,$ORIGIN/.."]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"C ABI smoke driver failed to build:\n{r.stderr[-4000:]}")
    return C_SMOKE_BIN


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
    print(build_c_smoke())
