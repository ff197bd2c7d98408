"""Tensor-level wrappers of the C ABI (device memory and streams come from torch).

``geom_scan``  -> holo_geom_scan_fwd : link rotations, prefix products, qh/kh/vh
``attention``  -> holo_attn_fwd      : causal attention, back-rotation
``attention_masked`` -> holo_attn_masked_fwd : any mask, causal (wrap through Hol) or inert mode
``attention_backward`` -> holo_attn_bwd : gradients of both wrt q, k, v and the generator
``attention_masked_train`` / ``attention_masked_backward`` -> holo_attn_masked_train_fwd /
    holo_attn_masked_bwd : the exact path's training forward (with its LSE) and gradient;
    with dropout_p > 0 holo_attn_masked_dropout_fwd / holo_attn_masked_dropout_bwd
``dropout_keep_mask`` -> holo_dropout_keep_mask : attention dropout's keep mask
``quat_to_dense`` -> holo_quat_to_dense
``add_layernorm`` -> holo_add_layernorm_fwd : residual add + LayerNorm of the decoder stack
``edge_hidden`` -> holo_edge_hidden_fwd : q/k/v and the interaction edge MLP's first layer
``edge_out``  -> holo_gemm_f32out_fwd : the edge MLP's last layer, fp32 output

Each wrapper checks devices, dtypes and strides on the host before the launch
(the kernels index exactly what these shapes describe), allocates its outputs
on the input's device and launches on the current HIP stream.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_DT = {torch.float32: _lib.HOLO_F32, torch.bfloat16: _lib.HOLO_BF16}
# operand types of the transported qh / kh / vh_t (fp16 only between the scan and holo_attn_fwd)
_OPDT = {**_DT, torch.float16: _lib.HOLO_F16}
# storage of P: name -> (holo_quat_format, torch dtype of the (B, H, T, nb, 4) tensor)
_PFMT = {"f32": (_lib.HOLO_QUAT_F32, torch.float32), "snorm16": (_lib.HOLO_QUAT_SNORM16, torch.int16)}
_MODE = {"causal": _lib.HOLO_MODE_CAUSAL, "inert": _lib.HOLO_MODE_INERT}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _one_gpu(what: str, *tensors: Optional[torch.Tensor]) -> torch.device:
    """The device of `tensors` (None entries skipped): every one must live on
    the same GPU, since the kernels dereference their data pointers as device
    addresses. Raises ValueError otherwise, before anything is launched."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError(f"{what}: every tensor must be on a GPU "
                             f"(got {t.device if isinstance(t, torch.Tensor) else type(t).__name__})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: all tensors must be on one device ({dev} and {t.device})")
    if dev is None:
        raise ValueError(f"{what}: no tensor given")
    return dev


def _token_view(t: torch.Tensor, B: int, T: int, H: int, width: int, name: str):
    """(B, T, H, width) view with unit inner stride and row-major (b, t) rows.
    Returns (row_stride, head_stride) in elements (row stride 0: one row
    broadcast to every token, strides (0, 0, hs, 1))."""
    if t.dim() != 4 or tuple(t.shape) != (B, T, H, width):
        raise ValueError(f"{name}: expected shape {(B, T, H, width)}, got {tuple(t.shape)}")
    sb, st, sh, sc = t.stride()
    if width > 1 and sc != 1:
        raise ValueError(f"{name}: needs unit inner stride (strides {t.stride()})")
    if sb == 0 and st == 0:
        return 0, (sh if H > 1 else width)
    hs = sh if H > 1 else width
    if T > 1:
        rs = st
        if B > 1 and sb != T * st:
            raise ValueError(f"{name}: (b, t) rows must be evenly strided (strides {t.stride()})")
    else:
        rs = sb if B > 1 else (H - 1) * hs + width
    return rs, hs


def token_rows_stride(x: torch.Tensor) -> Tuple[int, bool]:
    """(row stride in elements, is_view) of x.reshape(B*T, K) for x (B, T, K)
    with a unit last stride: a view when the (b, t) rows are evenly strided,
    otherwise torch copies into contiguous rows of stride K."""
    B, T, K = (int(n) for n in x.shape)
    if T == 1:
        return (int(x.stride(0)) if B > 1 else K), True
    if B == 1 or x.stride(0) == T * x.stride(1):
        return int(x.stride(1)), True
    return K, False


def padded_head_dim(d: int) -> int:
    return int(_lib.load().holo_padded_head_dim(d))


def padded_seq_len(T: int) -> int:
    return int(_lib.load().holo_padded_seq_len(T))


def qkvg_projection(x: torch.Tensor, w_qkv: torch.Tensor, w_gq: Optional[torch.Tensor],
                    w_gk: Optional[torch.Tensor]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """holo_qkvg_proj_fwd: x (B, T, K) bf16 -> qkv (B, T, n_qkv) bf16 = x w_qkv^T
    and g (B, T, n_gen) fp32 = x_t w_gq^T + x_{(t+1) mod T} w_gk^T (None when
    w_gq is None). Weights (n, K) bf16 (the nn.Linear layout)."""
    _one_gpu("qkvg_projection", x, w_qkv, w_gq, w_gk)
    lib = _lib.load()
    if x.dim() != 3 or x.dtype != torch.bfloat16:
        raise ValueError("qkvg_projection: x must be a (B, T, K) bfloat16 GPU tensor")
    B, T, K = (int(n) for n in x.shape)
    x2 = x.reshape(B * T, K)
    if x2.stride(1) != 1:
        raise ValueError("qkvg_projection: x rows must be contiguous")
    if (w_gq is None) != (w_gk is None):
        raise ValueError("qkvg_projection: w_gq and w_gk go together")
    ws = [w_qkv] + ([w_gq, w_gk] if w_gq is not None else [])
    for w in ws:
        if w.dtype != torch.bfloat16 or w.dim() != 2 or w.shape[1] != K or not w.is_contiguous() \
                or w.device != x.device:
            raise ValueError("qkvg_projection: weights must be contiguous (n, K) bfloat16 tensors on x's device")
    n_qkv = int(w_qkv.shape[0])
    n_gen = 0 if w_gq is None else int(w_gq.shape[0])
    if w_gq is not None and tuple(w_gk.shape) != tuple(w_gq.shape):
        raise ValueError("qkvg_projection: w_gq and w_gk must have one shape")
    qkv = torch.empty((B, T, n_qkv), dtype=torch.bfloat16, device=x.device)
    g = torch.empty((B, T, n_gen), dtype=torch.float32, device=x.device) if n_gen else None
    rc = lib.holo_qkvg_proj_fwd(B * T, T, K, n_qkv, n_gen, _ptr(x2), x2.stride(0), _ptr(w_qkv), _ptr(w_gq),
                                _ptr(w_gk), _ptr(qkv), n_qkv, _ptr(g), n_gen, _stream(x.device))
    _lib.check(rc, "holo_qkvg_proj_fwd")
    return qkv, g


def _bf16_weight(what: str, w: torch.Tensor, dev: torch.device, shape: Tuple[int, ...]) -> None:
    if w.dtype != torch.bfloat16 or tuple(w.shape) != shape or not w.is_contiguous() or w.device != dev:
        raise ValueError(f"{what}: expected a contiguous bfloat16 tensor of shape {shape} on {dev}, "
                         f"got {w.dtype} {tuple(w.shape)} on {w.device}")


def edge_hidden(x: torch.Tensor, w_qkv: Optional[torch.Tensor], w1: torch.Tensor, b1: torch.Tensor
                ) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """holo_edge_hidden_fwd: x (B, T, K) bf16 -> qkv (B, T, n_qkv) bf16 =
    x w_qkv^T (None when w_qkv is None) and hid (B, T, n_hid) bf16 =
    GELU([x_t ; x_{(t+1) mod T}] w1^T + b1), the interaction edge MLP's first
    layer (core/attention_fast_chunked.py:73-76) without the pair tensor.
    w1 (n_hid, 2K), b1 (n_hid), w_qkv (n_qkv, K): bf16, contiguous."""
    dev = _one_gpu("edge_hidden", x, w_qkv, w1, b1)
    lib = _lib.load()
    if x.dim() != 3 or x.dtype != torch.bfloat16:
        raise ValueError("edge_hidden: x must be a (B, T, K) bfloat16 GPU tensor")
    B, T, K = (int(n) for n in x.shape)
    x2 = x.reshape(B * T, K)
    if x2.stride(1) != 1:
        raise ValueError("edge_hidden: x rows must be contiguous")
    n_hid = int(w1.shape[0]) if w1.dim() == 2 else -1
    _bf16_weight("edge_hidden: w1", w1, dev, (n_hid, 2 * K))
    _bf16_weight("edge_hidden: b1", b1, dev, (n_hid,))
    n_qkv = 0
    if w_qkv is not None:
        n_qkv = int(w_qkv.shape[0]) if w_qkv.dim() == 2 else -1
        _bf16_weight("edge_hidden: w_qkv", w_qkv, dev, (n_qkv, K))
    qkv = torch.empty((B, T, n_qkv), dtype=torch.bfloat16, device=dev) if n_qkv else None
    hid = torch.empty((B, T, n_hid), dtype=torch.bfloat16, device=dev)
    rc = lib.holo_edge_hidden_fwd(B * T, T, K, n_qkv, n_hid, _ptr(x2), x2.stride(0), _ptr(w_qkv), _ptr(w1),
                                  2 * K, _ptr(b1), _ptr(qkv), n_qkv, _ptr(hid), n_hid, _stream(dev))
    _lib.check(rc, "holo_edge_hidden_fwd")
    return qkv, hid


def edge_out(hid: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """holo_gemm_f32out_fwd: hid (..., K) bf16 -> (..., N) fp32 = hid w2^T for
    w2 (N, K) bf16 contiguous, the edge MLP's last layer
    (core/attention_fast_chunked.py:76) with its sums kept in fp32 (no bias:
    the scan adds it per head)."""
    dev = _one_gpu("edge_out", hid, w2)
    lib = _lib.load()
    if hid.dtype != torch.bfloat16 or hid.dim() < 1:
        raise ValueError("edge_out: hid must be a bfloat16 GPU tensor")
    K = int(hid.shape[-1])
    a2 = hid.reshape(-1, K)
    if a2.stride(1) != 1:
        raise ValueError("edge_out: hid rows must be contiguous")
    N = int(w2.shape[0]) if w2.dim() == 2 else -1
    _bf16_weight("edge_out: w2", w2, dev, (N, K))
    c = torch.empty((*hid.shape[:-1], N), dtype=torch.float32, device=dev)
    M = int(a2.shape[0])
    if M == 0:
        return c
    rc = lib.holo_gemm_f32out_fwd(M, K, N, _ptr(a2), a2.stride(0), _ptr(w2), _ptr(c), N, _stream(dev))
    _lib.check(rc, "holo_gemm_f32out_fwd")
    return c


def geom_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gq: torch.Tensor,
              gk: Optional[torch.Tensor], edge_scale: float, want_hol: bool = False,
              p_format: str = "f32", mode: str = "causal", op_dtype: Optional[torch.dtype] = None,
              status: Optional[torch.Tensor] = None, static_scratch: bool = False
              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """q, k, v: (B,T,H,d) views; gq, gk: (B,T,H,3*nb) views (gk None: gq is the
    full link parameter g and a_t = edge_scale * g_t; gk with strides
    (0, 0, m, 1): a per-head constant, a_t = edge_scale * (gq_t + gk)). The generator may be
    fp32 with bf16 q/k/v (link parameters are composed in fp32 either way).
    Returns qh, kh (B,H,Tp,Dp), vh_t (B,H,Tp/64,Dp,64), P (B,H,T,nb,4) and
    Hol (B,H,nb,4) fp32 or None. P is fp32 quaternions (p_format "f32") or
    round(32767 q/|q|) as int16 ("snorm16", half the bytes; the attention
    epilogue uses either, quat_to_dense takes fp32). mode "causal" transports
    u^ = P^T u, "inert" u' = P u (for attention_masked in inert mode).
    op_dtype: type of qh/kh/vh_t (default q's dtype; float16 with bfloat16
    inputs for `attention`'s fp16 operands). status: an int32 device tensor
    of one element that receives the workspace status word (HOLO_WS_* bits,
    0 = clean) on the current stream. static_scratch: run
    holo_geom_scan_fwd_static, whose chained state lives in the library's
    per-device static array (no workspace; inputs whose state exceeds it
    raise NotImplementedError; calls that overlap on one device race)."""
    dev = _one_gpu("geom_scan", k, q, v, gq, gk, status)
    lib = _lib.load()
    B, T, H, d = k.shape
    nb = d // 3
    dt = k.dtype
    if dt not in _DT:
        raise ValueError(f"geom_scan: unsupported dtype {dt}")
    for name, t in (("q", q), ("v", v)):
        if t.dtype != dt or t.device != dev:
            raise ValueError(f"geom_scan: {name} must be {dt} on {dev}")
    gdt = gq.dtype
    if gdt not in _DT or (dt == torch.float32 and gdt != torch.float32):
        raise ValueError(f"geom_scan: generator dtype {gdt} with {dt} keys is not supported")
    for name, t in (("gq", gq), ("gk", gk)):
        if t is not None and (t.dtype != gdt or t.device != dev):
            raise ValueError(f"geom_scan: {name} must be {gdt} on {dev}")
    opdt = dt if op_dtype is None else op_dtype
    if opdt not in _OPDT or (dt == torch.float32) != (opdt == torch.float32):
        raise ValueError(f"geom_scan: operand dtype {opdt} with {dt} inputs is not supported")
    q_rs, q_hs = _token_view(q, B, T, H, d, "q")
    k_rs, k_hs = _token_view(k, B, T, H, d, "k")
    v_rs, v_hs = _token_view(v, B, T, H, d, "v")
    gq_rs, gq_hs = _token_view(gq, B, T, H, 3 * nb, "gq")
    if gq_rs == 0:
        raise ValueError("geom_scan: gq must have one row per token")
    gk_rs, gk_hs = (0, 0) if gk is None else _token_view(gk, B, T, H, 3 * nb, "gk")
    Dp, Tp = padded_head_dim(d), padded_seq_len(T)
    qh = torch.empty((B, H, Tp, Dp), dtype=opdt, device=dev)
    kh = torch.empty((B, H, Tp, Dp), dtype=opdt, device=dev)
    vh_t = torch.empty((B, H, Tp // 64, Dp, 64), dtype=opdt, device=dev)
    if p_format not in _PFMT:
        raise ValueError(f"geom_scan: p_format must be one of {sorted(_PFMT)}")
    if mode not in _MODE:
        raise ValueError(f"geom_scan: mode must be one of {sorted(_MODE)}")
    P = torch.empty((B, H, T, nb, 4), dtype=_PFMT[p_format][1], device=dev)
    hol = torch.empty((B, H, nb, 4), dtype=torch.float32, device=dev) if want_hol else None
    if static_scratch:
        if status is not None:
            raise ValueError("geom_scan: the static scratch has no status query")
        rc = lib.holo_geom_scan_fwd_static(
            B, T, H, d, _lib.HOLO_GEN_DIRECT if gk is None else _lib.HOLO_GEN_ADDITIVE,
            float(edge_scale), _DT[dt], _OPDT[opdt], _DT[gdt], _PFMT[p_format][0], _MODE[mode],
            _ptr(gq), gq_rs, gq_hs, _ptr(gk), gk_rs, gk_hs,
            _ptr(q), q_rs, q_hs, _ptr(k), k_rs, k_hs, _ptr(v), v_rs, v_hs,
            _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None, _ptr(hol), _stream(dev))
        _lib.check(rc, "holo_geom_scan_fwd_static")
        return qh, kh, vh_t, P, hol
    ws_bytes = int(lib.holo_geom_scan_workspace_size(B, T, H, d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    rc = lib.holo_geom_scan_fwd(
        B, T, H, d, _lib.HOLO_GEN_DIRECT if gk is None else _lib.HOLO_GEN_ADDITIVE,
        float(edge_scale), _DT[dt], _OPDT[opdt], _DT[gdt], _PFMT[p_format][0], _MODE[mode],
        _ptr(gq), gq_rs, gq_hs, _ptr(gk), gk_rs, gk_hs,
        _ptr(q), q_rs, q_hs, _ptr(k), k_rs, k_hs, _ptr(v), v_rs, v_hs,
        _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None, _ptr(hol),
        _ptr(ws), ws_bytes, _stream(dev))
    _lib.check(rc, "holo_geom_scan_fwd")
    if status is not None:
        workspace_status(ws, status)
    return qh, kh, vh_t, P, hol


def workspace_status(ws: torch.Tensor, status: torch.Tensor) -> None:
    """Copy the status word of a chained workspace (HOLO_WS_* bits) into
    `status`, an int32 device tensor of one element, on the current stream."""
    _one_gpu("workspace_status", ws, status)
    if status.dtype != torch.int32 or status.numel() != 1 or status.device != ws.device:
        raise ValueError("workspace_status: status must be a one-element int32 tensor on the workspace's device")
    rc = _lib.load().holo_workspace_status(_ptr(ws), ws.numel() * ws.element_size(), _ptr(status),
                                           _stream(ws.device))
    _lib.check(rc, "holo_workspace_status")


def attention(qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
              d: int, scale: float, out: Optional[torch.Tensor] = None,
              lse: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """qh, kh, vh_t, P from geom_scan for head dimension d.
    Returns o as a (B,T,H,d) tensor (contiguous (B,T,H*d) storage unless
    `out`, a (B,T,H,d) view, is given) of type out_dtype (default: fp32 for
    fp32 operands, bf16 for 16-bit ones; float32 is allowed with any
    operands). `lse`, a (B, H, Tp) fp32 tensor, receives each query's log2
    softmax normaliser (what `attention_backward` needs)."""
    _one_gpu("attention", qh, kh, vh_t, P, out, lse)
    lib = _lib.load()
    if P.dim() != 5:
        raise ValueError("attention: P must be (B, H, T, nb, 4)")
    B, H, T = (int(n) for n in P.shape[:3])
    nb = d // 3
    dev, dt = qh.device, qh.dtype
    if dev.type != "cuda" or dt not in _OPDT:
        raise ValueError(f"attention: qh must be a float32/bfloat16/float16 GPU tensor (got {dt} on {dev})")
    Dp, Tp = padded_head_dim(d), padded_seq_len(T)
    if tuple(qh.shape) != (B, H, Tp, Dp) or not qh.is_contiguous():
        raise ValueError("attention: qh does not match the geom_scan layout")
    if tuple(kh.shape) != (B, H, Tp, Dp) or not kh.is_contiguous() or kh.dtype != dt:
        raise ValueError("attention: kh does not match the geom_scan layout")
    if tuple(vh_t.shape) != (B, H, Tp // 64, Dp, 64) or not vh_t.is_contiguous() or vh_t.dtype != dt:
        raise ValueError("attention: vh_t does not match the geom_scan layout")
    pf = {torch.float32: _lib.HOLO_QUAT_F32, torch.int16: _lib.HOLO_QUAT_SNORM16}.get(P.dtype)
    if tuple(P.shape) != (B, H, T, nb, 4) or not P.is_contiguous() or pf is None:
        raise ValueError("attention: P does not match the geom_scan layout")
    for t in (kh, vh_t, P):
        if t.device != dev:
            raise ValueError("attention: all tensors must be on one device")
    odt = out.dtype if out is not None else out_dtype if out_dtype is not None else \
        (torch.float32 if dt == torch.float32 else torch.bfloat16)
    if odt not in _DT or (dt == torch.float32 and odt != torch.float32):
        raise ValueError(f"attention: output dtype {odt} with {dt} operands is not supported")
    if out is None:
        out = torch.empty((B, T, H, d), dtype=odt, device=dev)
    elif out.device != dev or (out_dtype is not None and out_dtype != out.dtype):
        raise ValueError("attention: out must be on qh's device (and of out_dtype when both are given)")
    o_rs, o_hs = _token_view(out, B, T, H, d, "out")
    if lse is not None and (tuple(lse.shape) != (B, H, Tp) or lse.dtype != torch.float32
                            or not lse.is_contiguous() or lse.device != dev):
        raise ValueError(f"attention: lse must be a contiguous fp32 {(B, H, Tp)} tensor on {dev}")
    rc = lib.holo_attn_fwd(B, T, H, d, _OPDT[dt], _DT[odt], pf, float(scale),
                           _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None,
                           _ptr(out), o_rs, o_hs, _ptr(lse), _stream(dev))
    _lib.check(rc, "holo_attn_fwd")
    return out


def _masked_inputs(what: str, qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
                   hol: Optional[torch.Tensor], d: int, mode: str, mask: Optional[torch.Tensor]):
    """Checks shared by the exact path's calls; returns (B, H, T, nb, device,
    dtype, holo_quat_format, uint8 mask or None, mask row stride)."""
    if mode not in _MODE:
        raise ValueError(f"{what}: mode must be one of {sorted(_MODE)}")
    if P.dim() != 5:
        raise ValueError(f"{what}: P must be (B, H, T, nb, 4)")
    B, H, T = (int(n) for n in P.shape[:3])
    nb = d // 3
    dev, dt = qh.device, qh.dtype
    if dev.type != "cuda" or dt not in _DT:
        raise ValueError(f"{what}: qh must be a float32/bfloat16 GPU tensor (got {dt} on {dev})")
    Dp, Tp = padded_head_dim(d), padded_seq_len(T)
    for name, t, shape in (("qh", qh, (B, H, Tp, Dp)), ("kh", kh, (B, H, Tp, Dp)),
                           ("vh_t", vh_t, (B, H, Tp // 64, Dp, 64))):
        if tuple(t.shape) != shape or not t.is_contiguous() or t.dtype != dt or t.device != dev:
            raise ValueError(f"{what}: {name} does not match the geom_scan layout")
    pf = {torch.float32: _lib.HOLO_QUAT_F32, torch.int16: _lib.HOLO_QUAT_SNORM16}.get(P.dtype)
    if tuple(P.shape) != (B, H, T, nb, 4) or not P.is_contiguous() or pf is None or P.device != dev:
        raise ValueError(f"{what}: P does not match the geom_scan layout")
    if mode == "causal" and nb:
        if hol is None or tuple(hol.shape) != (B, H, nb, 4) or hol.dtype != torch.float32 \
                or not hol.is_contiguous() or hol.device != dev:
            raise ValueError(f"{what}: causal mode needs hol, a contiguous fp32 (B, H, nb, 4) tensor")
    m8, m_rs = None, 0
    if mask is not None:
        if tuple(mask.shape) != (T, T) or mask.device != dev:
            raise ValueError(f"{what}: mask must be ({T}, {T}) on {dev}")
        m8 = mask.to(torch.bool).contiguous().view(torch.uint8)
        m_rs = T
    return B, H, T, nb, dev, dt, pf, m8, m_rs


def attention_masked(qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
                     hol: Optional[torch.Tensor], d: int, scale: float, mode: str = "causal",
                     mask: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention for any mask and either mode (the reference's exact path):
    qh, kh, vh_t, P from geom_scan in the same `mode`; hol (B, H, nb, 4) fp32
    (the scan's holonomy, needed in causal mode); mask (T, T) bool (True =
    allowed) or None (every pair allowed). A row that allows no key is NaN.
    Returns o as a (B,T,H,d) tensor, or writes `out`."""
    _one_gpu("attention_masked", qh, kh, vh_t, P, hol, mask, out)
    lib = _lib.load()
    B, H, T, nb, dev, dt, pf, m8, m_rs = _masked_inputs("attention_masked", qh, kh, vh_t, P, hol, d, mode, mask)
    if out is None:
        out = torch.empty((B, T, H, d), dtype=dt, device=dev)
    elif out.dtype != dt or out.device != dev:
        raise ValueError("attention_masked: out must match q's dtype and device")
    o_rs, o_hs = _token_view(out, B, T, H, d, "out")
    ws_bytes = int(lib.holo_attn_masked_workspace_size(B, T, H, d, _DT[dt], _MODE[mode], int(mask is not None)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    rc = lib.holo_attn_masked_fwd(B, T, H, d, _DT[dt], pf, _MODE[mode], float(scale),
                                  _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None,
                                  _ptr(hol) if mode == "causal" else None, _ptr(m8), m_rs,
                                  _ptr(out), o_rs, o_hs, _ptr(ws), ws_bytes, _stream(dev))
    _lib.check(rc, "holo_attn_masked_fwd")
    return out


def _dropout_args(what: str, dropout_p: float, seed: int, offset: int) -> Tuple[float, int, int]:
    p = float(dropout_p)
    if not (0.0 <= p < 1.0):
        raise ValueError(f"{what}: dropout_p must be in [0, 1), got {dropout_p}")
    seed, offset = int(seed), int(offset)
    if not (0 <= seed < 2 ** 64 and 0 <= offset < 2 ** 32):
        raise ValueError(f"{what}: seed must be a 64-bit and offset a 32-bit unsigned integer")
    return p, seed, offset


def dropout_keep_mask(B: int, T: int, H: int, dropout_p: float, seed: int, offset: int = 0,
                      device: Optional[torch.device] = None) -> torch.Tensor:
    """holo_dropout_keep_mask: (B, H, T, T) bool, True where attention dropout
    with (dropout_p, seed, offset) keeps pair (i, j) -- the mask that
    attention_masked_train and attention_masked_backward regenerate."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if dev.type != "cuda":
        raise ValueError("dropout_keep_mask: device must be a GPU")
    p, seed, offset = _dropout_args("dropout_keep_mask", dropout_p, seed, offset)
    keep = torch.empty((int(B), int(H), int(T), int(T)), dtype=torch.uint8, device=dev)
    if keep.numel() == 0:
        return keep.bool()
    with torch.cuda.device(dev):
        rc = _lib.load().holo_dropout_keep_mask(int(B), int(T), int(H), p, seed, offset, _ptr(keep), _stream(dev))
    _lib.check(rc, "holo_dropout_keep_mask")
    return keep.view(torch.bool)


def attention_masked_train(qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
                           hol: Optional[torch.Tensor], d: int, scale: float, mode: str = "causal",
                           mask: Optional[torch.Tensor] = None, dropout_p: float = 0.0, seed: int = 0,
                           offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """holo_attn_masked_train_fwd: attention_masked for training (P in fp32
    quaternions) that also returns each row's log2-domain log-sum-exp
    (B, H, Tp) fp32, which attention_masked_backward reads. Returns (o, lse).
    dropout_p > 0 runs holo_attn_masked_dropout_fwd: attention dropout on the
    softmax weights with the keep mask of (seed, offset); the backward must be
    given the same three values."""
    _one_gpu("attention_masked_train", qh, kh, vh_t, P, hol, mask)
    dropout_p, seed, offset = _dropout_args("attention_masked_train", dropout_p, seed, offset)
    lib = _lib.load()
    B, H, T, nb, dev, dt, pf, m8, m_rs = _masked_inputs("attention_masked_train", qh, kh, vh_t, P, hol, d, mode,
                                                        mask)
    if pf != _lib.HOLO_QUAT_F32:
        raise ValueError("attention_masked_train: P must be the fp32 quaternions")
    out = torch.empty((B, T, H, d), dtype=dt, device=dev)
    lse = torch.empty((B, H, padded_seq_len(T)), dtype=torch.float32, device=dev)
    o_rs, o_hs = _token_view(out, B, T, H, d, "out")
    ws_bytes = int(lib.holo_attn_masked_workspace_size(B, T, H, d, _DT[dt], _MODE[mode], int(mask is not None)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    tail = (_ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None, _ptr(hol) if mode == "causal" else None,
            _ptr(m8), m_rs, _ptr(out), o_rs, o_hs, _ptr(lse), _ptr(ws), ws_bytes, _stream(dev))
    if dropout_p > 0.0:
        rc = lib.holo_attn_masked_dropout_fwd(B, T, H, d, _DT[dt], _MODE[mode], float(scale), dropout_p, seed, offset,
                                              *tail)
        _lib.check(rc, "holo_attn_masked_dropout_fwd")
    else:
        rc = lib.holo_attn_masked_train_fwd(B, T, H, d, _DT[dt], _MODE[mode], float(scale), *tail)
        _lib.check(rc, "holo_attn_masked_train_fwd")
    return out, lse


def _bwd_inputs(what: str, gq, gk, qh, kh, vh_t, P, lse, o, dout, d, dq, dk, dv, dgq, dgk):
    """Checks shared by the backward calls; returns (B, H, T, nb, device,
    dtype, the five (row, head) strides of o, dout, dq, dk, dv, and those of
    gq, gk, dgq, dgk)."""
    B, H, T = (int(n) for n in P.shape[:3])
    dev, dt = qh.device, qh.dtype
    nb = d // 3
    m = 3 * nb
    Dp, Tp = padded_head_dim(d), padded_seq_len(T)
    if P.dtype != torch.float32 or tuple(P.shape) != (B, H, T, nb, 4) or not P.is_contiguous():
        raise ValueError(f"{what}: P must be the fp32 (B, H, T, nb, 4) quaternions")
    if tuple(qh.shape) != (B, H, Tp, Dp) or not qh.is_contiguous():
        raise ValueError(f"{what}: qh does not match the geom_scan layout")
    if tuple(kh.shape) != (B, H, Tp, Dp) or not kh.is_contiguous() or kh.dtype != dt:
        raise ValueError(f"{what}: kh does not match the geom_scan layout")
    if tuple(vh_t.shape) != (B, H, Tp // 64, Dp, 64) or not vh_t.is_contiguous() or vh_t.dtype != dt:
        raise ValueError(f"{what}: vh_t does not match the geom_scan layout")
    if tuple(lse.shape) != (B, H, Tp) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError(f"{what}: lse must be a contiguous fp32 (B, H, Tp) tensor")
    for t in (kh, vh_t, P, lse, o, dout, dq, dk, dv, gq, dgq) + tuple(x for x in (gk, dgk) if x is not None):
        if t.device != dev:
            raise ValueError(f"{what}: all tensors must be on one device")
    for name, t in (("o", o), ("dout", dout), ("dq", dq), ("dk", dk), ("dv", dv)):
        if t.dtype != dt:
            raise ValueError(f"{what}: {name} must be {dt}")
    for name, t in (("gq", gq), ("gk", gk), ("dgq", dgq), ("dgk", dgk)):
        if t is not None and t.dtype != torch.float32:
            raise ValueError(f"{what}: {name} must be float32")
    if (gk is None) != (dgk is None):
        raise ValueError(f"{what}: gk and dgk go together (additive generator)")
    views = [_token_view(t, B, T, H, d, n) for n, t in (("o", o), ("dout", dout), ("dq", dq), ("dk", dk), ("dv", dv))]
    gv = [(0, 0) if t is None else _token_view(t, B, T, H, m, n)
          for n, t in (("gq", gq), ("gk", gk), ("dgq", dgq), ("dgk", dgk))]
    return B, H, T, nb, dev, dt, views, gv


def _workspace(what: str, workspace: Optional[torch.Tensor], need: int, dev: torch.device) -> torch.Tensor:
    if workspace is not None and not workspace.is_contiguous():
        raise ValueError(f"{what}: workspace must be contiguous")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    return workspace


def attention_backward(gq: torch.Tensor, gk: Optional[torch.Tensor], edge_scale: float,
                       qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
                       lse: torch.Tensor, o: torch.Tensor, dout: torch.Tensor, d: int, scale: float,
                       dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor,
                       dgq: torch.Tensor, dgk: Optional[torch.Tensor],
                       workspace: Optional[torch.Tensor] = None) -> None:
    """Gradients of o = attention(geom_scan(q, k, v, gq, gk)) given dout = dL/do:
    writes dq, dk, dv ((B,T,H,d) views, dtype of o) and dgq, dgk ((B,T,H,m)
    fp32 views; gk/dgk None for the direct generator). P must be the fp32
    quaternions of the same forward, lse the normalisers its attention wrote."""
    _one_gpu("attention_backward", qh, kh, vh_t, P, lse, o, dout, dq, dk, dv, gq, gk, dgq, dgk, workspace)
    lib = _lib.load()
    B, H, T, nb, dev, dt, views, gv = _bwd_inputs("attention_backward", gq, gk, qh, kh, vh_t, P, lse, o, dout, d,
                                                  dq, dk, dv, dgq, dgk)
    need = int(lib.holo_attn_bwd_workspace_size(B, T, H, d, _DT[dt]))
    workspace = _workspace("attention_backward", workspace, need, dev)
    mode = _lib.HOLO_GEN_ADDITIVE if gk is not None else _lib.HOLO_GEN_DIRECT
    rc = lib.holo_attn_bwd(B, T, H, d, mode, float(edge_scale), _DT[dt], _lib.HOLO_F32, float(scale),
                           _ptr(gq), *gv[0], _ptr(gk), *gv[1],
                           _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None, _ptr(lse),
                           _ptr(o), *views[0], _ptr(dout), *views[1],
                           _ptr(dq), *views[2], _ptr(dk), *views[3], _ptr(dv), *views[4],
                           _ptr(dgq), *gv[2], _ptr(dgk), *gv[3],
                           _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(dev))
    _lib.check(rc, "holo_attn_bwd")


def attention_masked_backward(gq: torch.Tensor, gk: Optional[torch.Tensor], edge_scale: float,
                              qh: torch.Tensor, kh: torch.Tensor, vh_t: torch.Tensor, P: torch.Tensor,
                              hol: Optional[torch.Tensor], lse: torch.Tensor, o: torch.Tensor, dout: torch.Tensor,
                              d: int, scale: float, dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor,
                              dgq: torch.Tensor, dgk: Optional[torch.Tensor], mode: str = "causal",
                              mask: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                              dropout_p: float = 0.0, seed: int = 0, offset: int = 0) -> None:
    """holo_attn_masked_bwd: gradients of the exact path (any mask, either
    mode) given dout; arguments as attention_backward's, plus the mode, the
    holonomy hol (causal mode) and the mask of the forward; o and lse from
    attention_masked_train. In causal mode the closing edge (gq_{T-1}, gk_0)
    gets its gradient through the holonomy. dropout_p > 0 runs
    holo_attn_masked_dropout_bwd with the forward's dropout_p, seed, offset."""
    _one_gpu("attention_masked_backward", qh, kh, vh_t, P, hol, lse, o, dout, dq, dk, dv, gq, gk, dgq, dgk, mask,
             workspace)
    what = "attention_masked_backward"
    dropout_p, seed, offset = _dropout_args(what, dropout_p, seed, offset)
    lib = _lib.load()
    *_, m8, m_rs = _masked_inputs(what, qh, kh, vh_t, P, hol, d, mode, mask)
    B, H, T, nb, dev, dt, views, gv = _bwd_inputs(what, gq, gk, qh, kh, vh_t, P, lse, o, dout, d, dq, dk, dv, dgq, dgk)
    need = int(lib.holo_attn_masked_bwd_workspace_size(B, T, H, d, _DT[dt], _MODE[mode], int(mask is not None)))
    workspace = _workspace(what, workspace, need, dev)
    gm = _lib.HOLO_GEN_ADDITIVE if gk is not None else _lib.HOLO_GEN_DIRECT
    head = (B, T, H, d, gm, float(edge_scale), _DT[dt], _lib.HOLO_F32, _MODE[mode], float(scale))
    tail = (_ptr(gq), *gv[0], _ptr(gk), *gv[1],
            _ptr(qh), _ptr(kh), _ptr(vh_t), _ptr(P) if nb else None,
            _ptr(hol) if mode == "causal" else None, _ptr(lse), _ptr(m8), m_rs,
            _ptr(o), *views[0], _ptr(dout), *views[1],
            _ptr(dq), *views[2], _ptr(dk), *views[3], _ptr(dv), *views[4],
            _ptr(dgq), *gv[2], _ptr(dgk), *gv[3],
            _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(dev))
    if dropout_p > 0.0:
        rc = lib.holo_attn_masked_dropout_bwd(*head, dropout_p, seed, offset, *tail)
        _lib.check(rc, "holo_attn_masked_dropout_bwd")
    else:
        rc = lib.holo_attn_masked_bwd(*head, *tail)
        _lib.check(rc, "holo_attn_masked_bwd")


def quat_to_dense(quat: torch.Tensor, d: int) -> torch.Tensor:
    """(..., nb, 4) fp32 quaternions -> (..., d, d) fp32 block rotations."""
    _one_gpu("quat_to_dense", quat)
    lib = _lib.load()
    nb = d // 3
    if quat.shape[-2:] != (nb, 4) or quat.dtype != torch.float32 or not quat.is_contiguous():
        raise ValueError(f"quat_to_dense: expected contiguous fp32 (..., {nb}, 4)")
    lead = quat.shape[:-2]
    n = 1
    for s in lead:
        n *= int(s)
    out = torch.empty((*lead, d, d), dtype=torch.float32, device=quat.device)
    rc = lib.holo_quat_to_dense(n, d, _ptr(quat) if nb else None, _ptr(out), _stream(quat.device))
    _lib.check(rc, "holo_quat_to_dense")
    return out


def _bh_view(t: torch.Tensor, B: int, H: int, width: int, name: str) -> Tuple[int, int]:
    """(batch stride, head stride) of a (B, H, >= width) view with a unit last stride."""
    if t.dim() != 3 or t.shape[0] != B or t.shape[1] != H or t.shape[2] < width or t.stride(2) != 1:
        raise ValueError(f"{name}: expected a (B={B}, H={H}, {width}) view with a unit last stride")
    return t.stride(0), t.stride(1)


def decode_geom(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g_prev: Optional[torch.Tensor],
                gk: Optional[torch.Tensor], edge_scale: float, t: int, P: torch.Tensor,
                qh: torch.Tensor, kh_cache: torch.Tensor, vh_cache: torch.Tensor) -> None:
    """One decode step's geometry for token t (see holo_decode_geom_fwd).
    q, k, v: (B,H,d) views of the new token; g_prev: link parameters of token
    t-1 (B,H,3nb): gq in additive mode (with gk of token t), the edge-MLP
    output g in direct mode (gk None); not read when t = 0. P (B,H,nb,4) fp32
    is updated in place from P_{t-1} to P_t; qh (B,H,Dp) receives P_t^T q_t
    and row t of the caches the transported key and value."""
    _one_gpu("decode_geom", k, q, v, g_prev, gk, P, qh, kh_cache, vh_cache)
    lib = _lib.load()
    B, H, d = k.shape
    nb = d // 3
    dev, dt = k.device, k.dtype
    if dev.type != "cuda" or dt not in _DT:
        raise ValueError("decode_geom: k must be a float32/bfloat16 GPU tensor")
    Dp = padded_head_dim(d)
    cap = int(kh_cache.shape[2])
    if tuple(kh_cache.shape) != (B, H, cap, Dp) or not kh_cache.is_contiguous() or kh_cache.dtype != dt:
        raise ValueError("decode_geom: kh_cache must be a contiguous (B, H, capacity, Dp) tensor")
    if tuple(vh_cache.shape) != (B, H, cap // 64, Dp, 64) or not vh_cache.is_contiguous() or vh_cache.dtype != dt:
        raise ValueError("decode_geom: vh_cache must be a contiguous (B, H, capacity/64, Dp, 64) tensor")
    if tuple(qh.shape) != (B, H, Dp) or not qh.is_contiguous() or qh.dtype != dt:
        raise ValueError("decode_geom: qh must be a contiguous (B, H, Dp) tensor")
    if tuple(P.shape) != (B, H, nb, 4) or P.dtype != torch.float32 or not P.is_contiguous():
        raise ValueError("decode_geom: P must be a contiguous fp32 (B, H, nb, 4) tensor")
    q_s, k_s, v_s = (_bh_view(x, B, H, d, n) for x, n in ((q, "q"), (k, "k"), (v, "v")))
    gdt = torch.float32 if g_prev is None else g_prev.dtype
    if g_prev is not None and gdt not in _DT:
        raise ValueError("decode_geom: link parameters must be float32 or bfloat16")
    g_s = (0, 0) if g_prev is None else _bh_view(g_prev, B, H, 3 * nb, "g_prev")
    gk_s = (0, 0) if gk is None else _bh_view(gk, B, H, 3 * nb, "gk")
    mode = _lib.HOLO_GEN_ADDITIVE if gk is not None or (g_prev is None and t == 0) else _lib.HOLO_GEN_DIRECT
    rc = lib.holo_decode_geom_fwd(
        B, H, d, int(t), cap, mode, float(edge_scale), _DT[dt], _DT[gdt],
        _ptr(g_prev), g_s[0], g_s[1], _ptr(gk), gk_s[0], gk_s[1],
        _ptr(q), q_s[0], q_s[1], _ptr(k), k_s[0], k_s[1], _ptr(v), v_s[0], v_s[1],
        _ptr(P) if nb else None, _ptr(qh), _ptr(kh_cache), _ptr(vh_cache), _stream(dev))
    _lib.check(rc, "holo_decode_geom_fwd")


def decode_workspace_bytes(B: int, H: int, d: int, t: int) -> int:
    """Workspace bytes of decode_attention at position t."""
    return int(_lib.load().holo_decode_attn_workspace_size(B, H, d, int(t)))


def decode_attention(qh: torch.Tensor, kh_cache: torch.Tensor, vh_cache: torch.Tensor, P: torch.Tensor,
                     t: int, d: int, scale: float, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """o_t (B,H,d) = P_t sum_{j<=t} softmax_j(scale qh . kh_j) vh_j over cache rows 0..t
    (qh, the caches and P as decode_geom leaves them)."""
    dev = _one_gpu("decode_attention", qh, kh_cache, vh_cache, P, out, workspace)
    lib = _lib.load()
    dt = qh.dtype
    if dt not in _DT or qh.dim() != 3:
        raise ValueError("decode_attention: qh must be a (B, H, Dp) float32/bfloat16 tensor")
    B, H, Dp = (int(n) for n in qh.shape)
    nb = d // 3
    if Dp != padded_head_dim(d) or not qh.is_contiguous():
        raise ValueError(f"decode_attention: qh must be a contiguous (B, H, {padded_head_dim(d)}) tensor")
    cap = int(kh_cache.shape[2]) if kh_cache.dim() == 4 else -1
    if tuple(kh_cache.shape) != (B, H, cap, Dp) or not kh_cache.is_contiguous() or kh_cache.dtype != dt:
        raise ValueError("decode_attention: kh_cache must be a contiguous (B, H, capacity, Dp) tensor of qh's dtype")
    if tuple(vh_cache.shape) != (B, H, cap // 64, Dp, 64) or not vh_cache.is_contiguous() or vh_cache.dtype != dt:
        raise ValueError("decode_attention: vh_cache must be a contiguous (B, H, capacity/64, Dp, 64) tensor")
    if tuple(P.shape) != (B, H, nb, 4) or P.dtype != torch.float32 or not P.is_contiguous():
        raise ValueError("decode_attention: P must be a contiguous fp32 (B, H, nb, 4) tensor")
    if out is None:
        out = torch.empty((B, H, d), dtype=dt, device=dev)
    elif out.dtype != dt:
        raise ValueError("decode_attention: out must have qh's dtype")
    o_s = _bh_view(out, B, H, d, "out")
    need = int(lib.holo_decode_attn_workspace_size(B, H, d, int(t)))
    if workspace is not None and not workspace.is_contiguous():
        raise ValueError("decode_attention: workspace must be contiguous")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    rc = lib.holo_decode_attn_fwd(B, H, d, int(t), cap, _DT[dt], float(scale),
                                  _ptr(qh), _ptr(kh_cache), _ptr(vh_cache), _ptr(P) if nb else None,
                                  _ptr(out), o_s[0], o_s[1], _ptr(workspace),
                                  workspace.numel() * workspace.element_size(), _stream(dev))
    _lib.check(rc, "holo_decode_attn_fwd")
    return out


def add_layernorm(x: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                  eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """h = x + delta and y = LayerNorm(h) (weight, bias, eps over the last
    dimension) in one pass: the residual add and the next norm of a pre-LN
    decoder. Returns (h, y), both shaped like x."""
    _one_gpu("add_layernorm", x, delta, weight, bias)
    lib = _lib.load()
    if x.shape != delta.shape or x.dtype != delta.dtype or x.dtype not in _DT:
        raise ValueError("add_layernorm: x and delta must be GPU tensors of one shape and dtype (fp32/bf16)")
    d = int(x.shape[-1])
    if tuple(weight.shape) != (d,) or tuple(bias.shape) != (d,) or weight.dtype != x.dtype or bias.dtype != x.dtype:
        raise ValueError("add_layernorm: weight and bias must be (d,) tensors of x's dtype")
    x2, d2 = x.reshape(-1, d), delta.reshape(-1, d)
    if x2.stride(-1) != 1 or d2.stride(-1) != 1:
        raise ValueError("add_layernorm: rows must be contiguous")
    w, b = weight.contiguous(), bias.contiguous()
    h = torch.empty_like(x2)
    y = torch.empty_like(x2)
    rc = lib.holo_add_layernorm_fwd(x2.shape[0], d, _DT[x.dtype], float(eps), _ptr(x2), x2.stride(0),
                                    _ptr(d2), d2.stride(0), _ptr(w), _ptr(b), _ptr(h), h.stride(0),
                                    _ptr(y), y.stride(0), _stream(x.device))
    _lib.check(rc, "holo_add_layernorm_fwd")
    return h.view_as(x), y.view_as(x)
