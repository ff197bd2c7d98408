"""Python side of the CPU emulation of this package's kernels (test
infrastructure only).

``Emu`` loads tests/emu/_build/libholo_emu.so (the product HIP sources compiled
for x86-64 with AddressSanitizer, same C ABI as libholo_mi355x.so) and hands
out "device" buffers: guarded host allocations (inaccessible address space on
both sides, the tail of the last page poisoned) viewed as numpy arrays. A
kernel access outside any buffer stops the process with an AddressSanitizer
report naming the kernel source line, and a buffer resource whose range
leaves its allocation fails at the instruction that builds it.

The library needs the AddressSanitizer runtime loaded first, so emulated
runs happen in a child process: ``run_child(module, args)`` starts
``python -m <module> <args>`` with the runtime preloaded and returns its
exit status, its output and the JSON object on its last output line.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from tests.emu import build_emu  # noqa: E402

_P, _I, _L, _S = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t

STAT_NAMES = ["launches", "blocks", "lanes", "collectives", "mfma", "lds_dma", "partial_dword", "polls", "buffer_loads"]


def _abi_signatures():
    # the ABI's ctypes signatures, read from the package's binding module
    # without importing the package (which needs torch only for its wrappers)
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "_holo_lib_sigs", os.path.join(REPO, "holonomyawareattention_amd", "_lib.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class DevBuf:
    """A guarded allocation and its numpy view (`a`). bf16 data is stored as
    uint16 bit patterns."""

    def __init__(self, emu: "Emu", ptr: int, nbytes: int, shape, np_dtype):
        self.emu, self.ptr, self.nbytes = emu, ptr, nbytes
        raw = (ctypes.c_uint8 * max(nbytes, 1)).from_address(ptr)
        flat = np.frombuffer(raw, dtype=np.uint8, count=nbytes)
        self.a = flat.view(np_dtype).reshape(shape) if nbytes else np.zeros(shape, np_dtype)

    def free(self):
        if self.ptr:
            self.a = None
            self.emu.lib.emu_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16), for finite
    inputs (32-bit integer arithmetic, no wider temporaries)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u >> 16) & 1
    r += u
    r += 0x7FFF
    r >>= 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float64 values of x rounded to bf16 (through fp32, as torch rounds)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)


class Emu:
    def __init__(self, lib_path: Optional[str] = None, abi: bool = True):
        """lib_path: another emulated build (default: the product's);
        abi=False for a build that exports only the emu_* controls and its own
        entry points."""
        path = lib_path or build_emu.LIB
        self.lib = ctypes.CDLL(path)
        sigs = _abi_signatures()
        self.C = sigs
        for name, res, args in (sigs.SIGNATURES if abi else []):
            fn = getattr(self.lib, name)
            fn.restype, fn.argtypes = res, args
        L = self.lib
        L.emu_alloc.restype, L.emu_alloc.argtypes = _P, [_S]
        L.emu_free.restype, L.emu_free.argtypes = _I, [_P]
        L.emu_register.restype, L.emu_register.argtypes = None, [_P, _S]
        L.emu_set_sample.restype, L.emu_set_sample.argtypes = None, [_L, _L, _L]
        L.emu_set_lds_dma_mode.restype, L.emu_set_lds_dma_mode.argtypes = None, [_I]
        L.emu_set_log.restype, L.emu_set_log.argtypes = None, [_I]
        L.emu_log_text.restype, L.emu_log_text.argtypes = ctypes.c_char_p, []
        L.emu_stats.restype, L.emu_stats.argtypes = None, [ctypes.POINTER(ctypes.c_int64)]
        L.emu_reset_stats.restype, L.emu_reset_stats.argtypes = None, []

    # ---- buffers ----
    def empty(self, shape, dtype, mark: bool = True) -> DevBuf:
        """dtype: a numpy dtype, or "bf16" (stored as uint16). The bytes are
        set to 0xA5 (never a clean zero) unless mark=False (fresh pages read
        as zero)."""
        np_dt = np.dtype(np.uint16) if dtype == "bf16" else np.dtype(dtype)
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        n = int(np.prod(shape)) * np_dt.itemsize
        p = self.lib.emu_alloc(n)
        if not p:
            raise MemoryError(f"emu_alloc({n}) failed")
        buf = DevBuf(self, p, n, shape, np_dt)
        if n and mark:
            buf.a.reshape(-1).view(np.uint8)[:] = 0xA5        # marker: never a clean zero
        return buf

    def to_dev(self, x: np.ndarray, dtype) -> DevBuf:
        """Copy host data (any float array, or integers) into a new buffer of `dtype`."""
        b = self.empty(np.shape(x), dtype)
        if dtype == "bf16":
            b.a[...] = f32_to_bf16_bits(np.asarray(x, dtype=np.float32))
        else:
            b.a[...] = np.asarray(x).astype(b.a.dtype)
        return b

    @staticmethod
    def host(b: DevBuf, dtype=None) -> np.ndarray:
        """float64 copy of a buffer (bf16 decoded)."""
        if dtype == "bf16":
            return bf16_bits_to_f32(b.a).astype(np.float64)
        return b.a.astype(np.float64)

    # ---- control ----
    def sample(self, head: int = 0, tail: int = 0, stride: int = 0):
        """Run only workgroups [0, head), the last `tail` and every `stride`-th
        (0, 0, 0: all). For bounds checks of independent workgroups at full
        size; chained kernels need every workgroup."""
        self.lib.emu_set_sample(head, tail, stride)

    def lds_dma_mode(self, at_issue: bool):
        self.lib.emu_set_lds_dma_mode(1 if at_issue else 0)

    def log(self, on: bool = True):
        self.lib.emu_set_log(1 if on else 0)

    def log_text(self) -> str:
        return self.lib.emu_log_text().decode()

    def stats(self) -> Dict[str, int]:
        arr = (ctypes.c_int64 * 16)()
        self.lib.emu_stats(arr)
        return {n: int(arr[i]) for i, n in enumerate(STAT_NAMES)}

    def reset_stats(self):
        self.lib.emu_reset_stats()

    def check(self, rc: int, what: str):
        if rc != 0:
            raise RuntimeError(f"{what}: status {rc}: {self.lib.holo_last_error().decode()}")


def asan_env() -> Dict[str, str]:
    env = dict(os.environ)
    env["LD_PRELOAD"] = build_emu.ASAN_RT
    env["ASAN_OPTIONS"] = ("detect_leaks=0:halt_on_error=1:abort_on_error=1:handle_abort=1:"
                           "detect_stack_use_after_return=0:allocator_may_return_null=1:"
                           "detect_container_overflow=0:symbolize=1")
    env["ASAN_SYMBOLIZER_PATH"] = "/opt/rocm/llvm/bin/llvm-symbolizer"
    env["PYTHONPATH"] = REPO + os.pathsep + env.get("PYTHONPATH", "")
    env["OMP_NUM_THREADS"] = "1"
    return env


def _last_json(stdout: str) -> Optional[dict]:
    for line in reversed(stdout.splitlines()):
        line = line.strip()
        if line.startswith("{"):
            try:
                return json.loads(line)
            except json.JSONDecodeError:
                continue
    return None


class Child:
    """A started emulated run (see run_child); wait() returns the same triple."""

    def __init__(self, module: str, args: Sequence[str], timeout: float):
        self.timeout = timeout
        self.p = subprocess.Popen([sys.executable, "-m", module, *args], cwd=REPO, env=asan_env(),
                                  stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
        self.done = None

    def wait(self) -> Tuple[int, str, Optional[dict]]:
        if self.done is None:
            try:
                out, err = self.p.communicate(timeout=self.timeout)
            except subprocess.TimeoutExpired:
                self.p.kill()
                out, err = self.p.communicate()
                err += f"\n[emulated run killed after {self.timeout} s]"
            self.done = (self.p.returncode, out + err, _last_json(out))
        return self.done


def start_child(module: str, args: Sequence[str], timeout: float = 900) -> Child:
    build_emu.build()
    return Child(module, args, timeout)


def run_child(module: str, args: Sequence[str], timeout: float = 900) -> Tuple[int, str, Optional[dict]]:
    """Run `python -m module args...` under AddressSanitizer; returns (exit
    status, combined output, the JSON object printed on the last line that
    parses as one, or None)."""
    build_emu.build()
    r = subprocess.run([sys.executable, "-m", module, *args], cwd=REPO, env=asan_env(), capture_output=True,
                       text=True, timeout=timeout)
    out = r.stdout + r.stderr
    res = None
    for line in reversed(r.stdout.splitlines()):
        line = line.strip()
        if line.startswith("{"):
            try:
                res = json.loads(line)
                break
            except json.JSONDecodeError:
                continue
    return r.returncode, out, res
