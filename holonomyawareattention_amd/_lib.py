"""ctypes binding of libholo_mi355x.so (the C ABI in include/holo_mi355x.h).

The library is built in-tree by ``python -m holonomyawareattention_amd.build``
(or ``__graft_entry__.build()``). There is no fallback: if the library is
missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libholo_mi355x.so")

HOLO_OK = 0
HOLO_ERR_INVALID_ARG = 1
HOLO_ERR_BAD_SHAPE = 2
HOLO_ERR_UNSUPPORTED = 3
HOLO_ERR_WORKSPACE = 4
HOLO_ERR_LAUNCH = 5

HOLO_F32 = 0
HOLO_BF16 = 1
HOLO_F16 = 2

HOLO_WS_TIMEOUT = 1
HOLO_WS_OVERFLOW = 2

HOLO_SCAN_STATIC_SCRATCH_BYTES = 32 << 20   # holo_geom_scan_fwd_static's per-device state array

HOLO_GEN_ADDITIVE = 0
HOLO_GEN_DIRECT = 1

HOLO_QUAT_F32 = 0
HOLO_QUAT_SNORM16 = 1

HOLO_MODE_CAUSAL = 0
HOLO_MODE_INERT = 1

# (name, restype, argtypes) for every exported symbol of the header
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
SIGNATURES = [
    ("holo_last_error", ctypes.c_char_p, []),
    ("holo_abi_version", _I, []),
    ("holo_padded_head_dim", _I, [_I]),
    ("holo_padded_seq_len", _L, [_L]),
    ("holo_qkvg_proj_fwd", _I, [_L, _L, _I, _I, _I, _P, _L, _P, _P, _P, _P, _L, _P, _L, _P]),
    ("holo_edge_hidden_fwd", _I, [_L, _L, _I, _I, _I, _P, _L, _P, _P, _L, _P, _P, _L, _P, _L, _P]),
    ("holo_gemm_f32out_fwd", _I, [_L, _I, _I, _P, _L, _P, _P, _L, _P]),
    ("holo_geom_scan_workspace_size", _S, [_I, _L, _I, _I]),
    ("holo_workspace_status", _I, [_P, _S, _P, _P]),
    ("holo_geom_scan_fwd", _I, [_I, _L, _I, _I, _I, _F, _I, _I, _I, _I, _I,
                                _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L,
                                _P, _P, _P, _P, _P, _P, _S, _P]),
    ("holo_geom_scan_fwd_static", _I, [_I, _L, _I, _I, _I, _F, _I, _I, _I, _I, _I,
                                       _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L,
                                       _P, _P, _P, _P, _P, _P]),
    ("holo_attn_fwd", _I, [_I, _L, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _L, _L, _P, _P]),
    ("holo_attn_masked_workspace_size", _S, [_I, _L, _I, _I, _I, _I, _I]),
    ("holo_attn_masked_fwd", _I, [_I, _L, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _L,
                                  _P, _L, _L, _P, _S, _P]),
    ("holo_attn_masked_train_fwd", _I, [_I, _L, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _L,
                                        _P, _L, _L, _P, _P, _S, _P]),
    ("holo_attn_bwd_workspace_size", _S, [_I, _L, _I, _I, _I]),
    ("holo_attn_bwd", _I, [_I, _L, _I, _I, _I, _F, _I, _I, _F,
                           _P, _L, _L, _P, _L, _L,
                           _P, _P, _P, _P, _P,
                           _P, _L, _L, _P, _L, _L,
                           _P, _L, _L, _P, _L, _L, _P, _L, _L,
                           _P, _L, _L, _P, _L, _L,
                           _P, _S, _P]),
    ("holo_attn_masked_bwd_workspace_size", _S, [_I, _L, _I, _I, _I, _I, _I]),
    ("holo_attn_masked_bwd", _I, [_I, _L, _I, _I, _I, _F, _I, _I, _I, _F,
                                  _P, _L, _L, _P, _L, _L,
                                  _P, _P, _P, _P, _P, _P, _P, _L,
                                  _P, _L, _L, _P, _L, _L,
                                  _P, _L, _L, _P, _L, _L, _P, _L, _L,
                                  _P, _L, _L, _P, _L, _L,
                                  _P, _S, _P]),
    ("holo_attn_masked_dropout_fwd", _I, [_I, _L, _I, _I, _I, _I, _F, _F, _U64, _U32, _P, _P, _P, _P, _P, _P, _L,
                                          _P, _L, _L, _P, _P, _S, _P]),
    ("holo_attn_masked_dropout_bwd", _I, [_I, _L, _I, _I, _I, _F, _I, _I, _I, _F, _F, _U64, _U32,
                                          _P, _L, _L, _P, _L, _L,
                                          _P, _P, _P, _P, _P, _P, _P, _L,
                                          _P, _L, _L, _P, _L, _L,
                                          _P, _L, _L, _P, _L, _L, _P, _L, _L,
                                          _P, _L, _L, _P, _L, _L,
                                          _P, _S, _P]),
    ("holo_dropout_keep_mask", _I, [_I, _L, _I, _F, _U64, _U32, _P, _P]),
    ("holo_quat_to_dense", _I, [_L, _I, _P, _P, _P]),
    ("holo_add_layernorm_fwd", _I, [_L, _I, _I, _F, _P, _L, _P, _L, _P, _P, _P, _L, _P, _L, _P]),
    ("holo_decode_geom_fwd", _I, [_I, _I, _I, _L, _L, _I, _F, _I, _I,
                                  _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L,
                                  _P, _P, _P, _P, _P]),
    ("holo_decode_attn_workspace_size", _S, [_I, _I, _I, _L]),
    ("holo_decode_attn_fwd", _I, [_I, _I, _I, _L, _L, _I, _F, _P, _P, _P, _P, _P, _L, _L, _P, _S, _P]),
]

_lib = None


class HoloError(RuntimeError):
    """Raised for launch failures and invalid arguments reported by the library."""


def load() -> ctypes.CDLL:
    """Load the shared library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 HIP library with "
                "`python -m holonomyawareattention_amd.build` (there is no fallback path)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a holo_status to the exception types the reference raises."""
    if rc == HOLO_OK:
        return
    msg = f"{what}: {load().holo_last_error().decode(errors='replace')}"
    if rc == HOLO_ERR_BAD_SHAPE:
        raise ValueError(msg)
    if rc == HOLO_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise HoloError(f"{msg} (status {rc})")
