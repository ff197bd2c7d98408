/* The C form of one training step's core on the exact path (any mask, causal
 * mode through the holonomy or inert mode; off in the module by default):
 * the training forward with its per-row log-sum-exp, then the backward,
 * from the scan's outputs (P as fp32 quaternions, hol in causal mode) to
 * dq, dk, dv and the additive generator's dgq, dgk (and the same with
 * attention dropout). Every buffer is the
 * caller's; the two workspaces come from their *_workspace_size queries:
 *   q, k, v, o, dout, dq, dk, dv  bf16, (b, t, h, c) at ptr[(b*T + t)*rs + h*hs + c]
 *   gq, gk, dgq, dgk             fp32, (b, t, h, j) at ptr[(b*T + t)*g_rs + h*g_hs + j]
 *   lse                          fp32 (B, H, Tp)
 *   mask                         uint8 (T, T), nonzero = allowed, or NULL
 * Compiled by the library build (a stale signature fails there); not run. */
#include <math.h>
#include <stdio.h>

#include "holo_mi355x.h"

int holo_example_exact_train_bf16(int B, int64_t T, int H, int d, int mode, float edge_scale,
                                  const float* gq, const float* gk, int64_t g_rs, int64_t g_hs,
                                  const void* qh, const void* kh, const void* vh_t, const float* P,
                                  const float* hol, const uint8_t* mask,
                                  void* o, float* lse, const void* dout,
                                  void* dq, void* dk, void* dv, int64_t qkv_rs, int64_t qkv_hs,
                                  float* dgq, float* dgk,
                                  void* fwd_ws, size_t fwd_ws_bytes, void* bwd_ws, size_t bwd_ws_bytes,
                                  void* stream) {
  const float scale = 1.0f / sqrtf((float)d);
  const int64_t mask_rs = mask ? T : 0;
  int rc = holo_attn_masked_train_fwd(B, T, H, d, HOLO_BF16, mode, scale, qh, kh, vh_t, P, hol, mask, mask_rs,
                                      o, (int64_t)H * d, d, lse, fwd_ws, fwd_ws_bytes, stream);
  if (rc == HOLO_OK)
    rc = holo_attn_masked_bwd(B, T, H, d, HOLO_GEN_ADDITIVE, edge_scale, HOLO_BF16, HOLO_F32, mode, scale,
                              gq, g_rs, g_hs, gk, g_rs, g_hs, qh, kh, vh_t, P, hol, lse, mask, mask_rs,
                              o, (int64_t)H * d, d, dout, (int64_t)H * d, d,
                              dq, qkv_rs, qkv_hs, dk, qkv_rs, qkv_hs, dv, qkv_rs, qkv_hs,
                              dgq, g_rs, g_hs, dgk, g_rs, g_hs, bwd_ws, bwd_ws_bytes, stream);
  if (rc != HOLO_OK) fprintf(stderr, "holo: %s\n", holo_last_error());
  return rc;
}

/* The same step with attention dropout (probability p, 0 <= p < 1): the
 * backward regenerates the forward's keep mask from the same p, seed and
 * offset, so the three go to both calls. */
int holo_example_exact_train_dropout_bf16(int B, int64_t T, int H, int d, int mode, float edge_scale, float p,
                                          uint64_t seed, uint32_t offset,
                                          const float* gq, const float* gk, int64_t g_rs, int64_t g_hs,
                                          const void* qh, const void* kh, const void* vh_t, const float* P,
                                          const float* hol, const uint8_t* mask,
                                          void* o, float* lse, const void* dout,
                                          void* dq, void* dk, void* dv, int64_t qkv_rs, int64_t qkv_hs,
                                          float* dgq, float* dgk,
                                          void* fwd_ws, size_t fwd_ws_bytes, void* bwd_ws, size_t bwd_ws_bytes,
                                          void* stream) {
  const float scale = 1.0f / sqrtf((float)d);
  const int64_t mask_rs = mask ? T : 0;
  int rc = holo_attn_masked_dropout_fwd(B, T, H, d, HOLO_BF16, mode, scale, p, seed, offset, qh, kh, vh_t, P, hol,
                                        mask, mask_rs, o, (int64_t)H * d, d, lse, fwd_ws, fwd_ws_bytes, stream);
  if (rc == HOLO_OK)
    rc = holo_attn_masked_dropout_bwd(B, T, H, d, HOLO_GEN_ADDITIVE, edge_scale, HOLO_BF16, HOLO_F32, mode, scale,
                                      p, seed, offset, gq, g_rs, g_hs, gk, g_rs, g_hs, qh, kh, vh_t, P, hol, lse,
                                      mask, mask_rs, o, (int64_t)H * d, d, dout, (int64_t)H * d, d,
                                      dq, qkv_rs, qkv_hs, dk, qkv_rs, qkv_hs, dv, qkv_rs, qkv_hs,
                                      dgq, g_rs, g_hs, dgk, g_rs, g_hs, bwd_ws, bwd_ws_bytes, stream);
  if (rc != HOLO_OK) fprintf(stderr, "holo: %s\n", holo_last_error());
  return rc;
}
