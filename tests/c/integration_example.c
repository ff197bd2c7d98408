/* The C form of the binding: one layer core on the bf16 path, from the
 * projections' outputs to the per-head attention output o (what the
 * reference's run_fwd_kernel computes, kernel/attention_kernel.py:122-134,
 * plus the geometry of core/attention_fast_chunked.py:73-110). The caller
 * owns every buffer:
 *   q, k, v   bf16, element (b, t, h, c) at ptr[(b*T + t)*qkv_rs + h*qkv_hs + c]
 *   gq, gk    fp32 generator outputs, (b, t, h, j) at ptr[(b*T + t)*g_rs + h*g_hs + j]
 *   qh, kh    2 * B*H*Tp*Dp fp16 each, vh_t B*H*Tp*Dp fp16 (Tp, Dp: padded sizes)
 *   P         B*H*T*(d/3)*4 int16, ws holo_geom_scan_workspace_size(B, T, H, d) bytes
 *   o         out_dtype (HOLO_BF16 or HOLO_F32), (B, T, H, d) contiguous
 */
#include <math.h>
#include <stdio.h>

#include "holo_mi355x.h"

int holo_example_core_bf16(int B, int64_t T, int H, int d, float edge_scale,
                           const void* gq, const void* gk, int64_t g_rs, int64_t g_hs,
                           const void* q, const void* k, const void* v, int64_t qkv_rs, int64_t qkv_hs,
                           void* qh, void* kh, void* vh_t, void* P, void* ws, size_t ws_bytes,
                           void* o, int out_dtype, void* stream) {
  int rc = holo_geom_scan_fwd(B, T, H, d, HOLO_GEN_ADDITIVE, edge_scale, HOLO_BF16, HOLO_F16, HOLO_F32,
                              HOLO_QUAT_SNORM16, HOLO_MODE_CAUSAL,
                              gq, g_rs, g_hs, gk, g_rs, g_hs,
                              q, qkv_rs, qkv_hs, k, qkv_rs, qkv_hs, v, qkv_rs, qkv_hs,
                              qh, kh, vh_t, P, /*hol*/ NULL, ws, ws_bytes, stream);
  if (rc == HOLO_OK)
    rc = holo_attn_fwd(B, T, H, d, HOLO_F16, out_dtype, HOLO_QUAT_SNORM16, 1.0f / sqrtf((float)d),
                       qh, kh, vh_t, P, o, /*row stride*/ (int64_t)H * d, /*head stride*/ d,
                       /*lse*/ NULL, stream);
  if (rc != HOLO_OK) fprintf(stderr, "holo: %s\n", holo_last_error());
  return rc;
}
