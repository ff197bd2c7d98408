# kernel/attention_kernel_mi355x.py -- the binding a maintainer would add to the
# reference next to kernel/attention_kernel.py (its operator boundary,
# run_fwd_kernel, kernel/attention_kernel.py:122-134): the MI355X library
# through ctypes, torch for device memory and the stream.
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("HOLO_MI355X_LIB",
                          os.path.join(_HERE, "..", "..", "holonomyawareattention_amd", "libholo_mi355x.so"))
lib = ctypes.CDLL(LIB_PATH)
P_, L_, I_, F_, S_ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
# holo_geom_scan_fwd(B, T, H, d, gen_mode, edge_scale, io_dtype, op_dtype, gen_dtype, p_format, mode,
#                    gq, gk, q, k, v (pointer, row stride, head stride each),
#                    qh, kh, vh_t, P, hol, workspace, workspace_bytes, stream)
lib.holo_geom_scan_fwd.argtypes = [I_, L_, I_, I_, I_, F_, I_, I_, I_, I_, I_] + [P_, L_, L_] * 5 + [P_] * 6 + [S_, P_]
# holo_attn_fwd(B, T, H, d, op_dtype, out_dtype, p_format, scale, qh, kh, vh_t, P,
#               o, o_row_stride, o_head_stride, lse, stream)
lib.holo_attn_fwd.argtypes = [I_, L_, I_, I_, I_, I_, I_, F_, P_, P_, P_, P_, P_, L_, L_, P_, P_]
lib.holo_geom_scan_workspace_size.argtypes = [I_, L_, I_, I_]
lib.holo_geom_scan_workspace_size.restype = S_
lib.holo_last_error.restype = ctypes.c_char_p
HOLO_F32, HOLO_BF16, HOLO_F16 = 0, 1, 2
HOLO_GEN_ADDITIVE = 0
HOLO_QUAT_F32, HOLO_QUAT_SNORM16 = 0, 1
HOLO_MODE_CAUSAL = 0


def run_fwd_kernel_mi355x(q, k, v, gq, gk, edge_scale, scale, out_dtype=None):
    """q, k, v: (B,T,H,d) views of the qkv projection (bf16 or fp32); gq, gk:
    (B,T,H,3*(d//3)) fp32 views of the generator projection. Returns o
    (B,T,H,d) = P_i sum_j softmax_j(scale qh_i.kh_j) vh_j, in q's dtype unless
    out_dtype is given (torch.float32 is allowed with bf16 inputs)."""
    B, T, H, d = q.shape
    nb, Dp, Tp = d // 3, (d + 31) // 32 * 32, (T + 63) // 64 * 64
    dev, dt = q.device, q.dtype
    bf16 = dt == torch.bfloat16
    # transported q/k/v: fp16 operands on the bf16 path (11-bit significands at
    # the bf16 matrix-core rate), fp32 otherwise
    opdt, op = (torch.float16, HOLO_F16) if bf16 else (torch.float32, HOLO_F32)
    io = HOLO_BF16 if bf16 else HOLO_F32
    qh = torch.empty(B, H, Tp, Dp, dtype=opdt, device=dev)
    kh = torch.empty_like(qh)
    vh_t = torch.empty(B, H, Tp // 64, Dp, 64, dtype=opdt, device=dev)
    # P between the two calls: int16 quaternions on the bf16 path (8 bytes each)
    pf = HOLO_QUAT_SNORM16 if bf16 else HOLO_QUAT_F32
    Pq = torch.empty(B, H, T, nb, 4, dtype=torch.int16 if bf16 else torch.float32, device=dev)
    ws_n = lib.holo_geom_scan_workspace_size(B, T, H, d)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    rs = lambda t: t.stride(1)            # token-row stride (elements)
    hs = lambda t: t.stride(2)            # head stride (elements)
    rc = lib.holo_geom_scan_fwd(B, T, H, d, HOLO_GEN_ADDITIVE, edge_scale, io, op, HOLO_F32, pf, HOLO_MODE_CAUSAL,
                                gq.data_ptr(), rs(gq), hs(gq), gk.data_ptr(), rs(gk), hs(gk),
                                q.data_ptr(), rs(q), hs(q), k.data_ptr(), rs(k), hs(k),
                                v.data_ptr(), rs(v), hs(v),
                                qh.data_ptr(), kh.data_ptr(), vh_t.data_ptr(), Pq.data_ptr(), None,
                                ws.data_ptr(), ws_n, s)
    if rc:
        raise RuntimeError(lib.holo_last_error().decode())
    odt = out_dtype or dt
    o = torch.empty(B, T, H, d, dtype=odt, device=dev)
    rc = lib.holo_attn_fwd(B, T, H, d, op, HOLO_F32 if odt == torch.float32 else HOLO_BF16, pf, scale,
                           qh.data_ptr(), kh.data_ptr(), vh_t.data_ptr(), Pq.data_ptr(),
                           o.data_ptr(), H * d, d, None, s)
    if rc:
        raise RuntimeError(lib.holo_last_error().decode())
    return o
