/*
 * A C caller of the library with no PyTorch: HIP runtime allocations,
 * holo_geom_scan_fwd + holo_attn_fwd (the causal tril path) and
 * holo_attn_masked_fwd (the ring mask, causal mode) on fp32 inputs read from
 * files, the bf16 path through holo_example_core_bf16 (tests/c/
 * integration_example.c, the documented C binding example) on the same
 * inputs rounded to bf16, outputs written to files; plus the error path of a
 * bad call and the scan's workspace status.
 *
 *   abi_smoke <dir> B T H d edge_scale
 * reads  <dir>/{q,k,v,gq,gk}.f32 (B, T, H, d|3*(d/3)) row-major fp32,
 * writes <dir>/o_tril.f32, <dir>/o_ring.f32 and <dir>/o_bf16.f32 (B, T, H, d)
 * fp32. Exit status 0 on success; the first failure is printed.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "holo_mi355x.h"

int holo_example_core_bf16(int B, int64_t T, int H, int d, float edge_scale,
                           const void* gq, const void* gk, int64_t g_rs, int64_t g_hs,
                           const void* q, const void* k, const void* v, int64_t qkv_rs, int64_t qkv_hs,
                           void* qh, void* kh, void* vh_t, void* P, void* ws, size_t ws_bytes,
                           void* o, int out_dtype, void* stream);

/* round-to-nearest-even fp32 -> bf16 bits (finite inputs) */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int die(const char* what, const char* detail) {
  fprintf(stderr, "abi_smoke: %s: %s\n", what, detail);
  return 1;
}

static float* read_file(const char* dir, const char* name, size_t n) {
  char path[1024];
  snprintf(path, sizeof(path), "%s/%s", dir, name);
  FILE* f = fopen(path, "rb");
  if (!f) return NULL;
  float* buf = (float*)malloc(n * sizeof(float));
  size_t got = buf ? fread(buf, sizeof(float), n, f) : 0;
  fclose(f);
  if (got != n) { free(buf); return NULL; }
  return buf;
}

static int write_file(const char* dir, const char* name, const float* buf, size_t n) {
  char path[1024];
  snprintf(path, sizeof(path), "%s/%s", dir, name);
  FILE* f = fopen(path, "wb");
  if (!f) return 1;
  size_t put = fwrite(buf, sizeof(float), n, f);
  fclose(f);
  return put != n;
}

static void* dev_alloc(size_t bytes) {
  void* p = NULL;
  return hipMalloc(&p, bytes ? bytes : 16) == hipSuccess ? p : NULL;
}

int main(int argc, char** argv) {
  if (argc != 7) return die("usage", "abi_smoke <dir> B T H d edge_scale");
  const char* dir = argv[1];
  const int B = atoi(argv[2]), H = atoi(argv[4]), d = atoi(argv[5]);
  const int64_t T = atoll(argv[3]);
  const float es = (float)atof(argv[6]);
  const int nb = d / 3, m = 3 * nb;
  const int64_t Tp = holo_padded_seq_len(T);
  const int Dp = holo_padded_head_dim(d);
  const size_t n_io = (size_t)B * T * H * d, n_g = (size_t)B * T * H * m;

  /* the error path: status code and message, nothing launched */
  if (holo_attn_fwd(0, T, H, d, HOLO_F32, HOLO_F32, HOLO_QUAT_F32, 0.1f, NULL, NULL, NULL, NULL, NULL, 0, 0, NULL,
                    NULL) !=
          HOLO_ERR_BAD_SHAPE ||
      strlen(holo_last_error()) == 0)
    return die("error path", "B = 0 did not report HOLO_ERR_BAD_SHAPE with a message");

  float* hq = read_file(dir, "q.f32", n_io);
  float* hk = read_file(dir, "k.f32", n_io);
  float* hv = read_file(dir, "v.f32", n_io);
  float* hgq = read_file(dir, "gq.f32", n_g);
  float* hgk = read_file(dir, "gk.f32", n_g);
  if (!hq || !hk || !hv || !hgq || !hgk) return die("inputs", "missing or short input file");

  float *q = dev_alloc(n_io * 4), *k = dev_alloc(n_io * 4), *v = dev_alloc(n_io * 4);
  float *gq = dev_alloc(n_g * 4), *gk = dev_alloc(n_g * 4);
  const size_t n_path = (size_t)B * H * Tp * Dp;
  float *qh = dev_alloc(n_path * 4), *kh = dev_alloc(n_path * 4), *vh_t = dev_alloc(n_path * 4);
  float *P = dev_alloc((size_t)B * H * T * nb * 16), *hol = dev_alloc((size_t)B * H * nb * 16);
  float *o = dev_alloc(n_io * 4), *o2 = dev_alloc(n_io * 4);
  const size_t ws_bytes = holo_geom_scan_workspace_size(B, T, H, d);
  void* ws = dev_alloc(ws_bytes);
  const size_t mws_bytes = holo_attn_masked_workspace_size(B, T, H, d, HOLO_F32, HOLO_MODE_CAUSAL, 1);
  void* mws = dev_alloc(mws_bytes);
  uint8_t* mask = dev_alloc((size_t)T * T);
  if (!q || !k || !v || !gq || !gk || !qh || !kh || !vh_t || !P || !hol || !o || !o2 || !ws || !mws || !mask)
    return die("hipMalloc", "allocation failed");
  uint8_t* hmask = (uint8_t*)calloc((size_t)T * T, 1);
  for (int64_t i = 0; i < T; ++i) {                 /* ring mask: i-1, i, i+1 (mod T) */
    hmask[i * T + i] = 1;
    hmask[i * T + (i + T - 1) % T] = 1;
    hmask[i * T + (i + 1) % T] = 1;
  }
  if (hipMemcpy(q, hq, n_io * 4, hipMemcpyHostToDevice) || hipMemcpy(k, hk, n_io * 4, hipMemcpyHostToDevice) ||
      hipMemcpy(v, hv, n_io * 4, hipMemcpyHostToDevice) || hipMemcpy(gq, hgq, n_g * 4, hipMemcpyHostToDevice) ||
      hipMemcpy(gk, hgk, n_g * 4, hipMemcpyHostToDevice) ||
      hipMemcpy(mask, hmask, (size_t)T * T, hipMemcpyHostToDevice))
    return die("hipMemcpy", "upload failed");

  const float scale = 1.0f / sqrtf((float)d);
  int rc = holo_geom_scan_fwd(B, T, H, d, HOLO_GEN_ADDITIVE, es, HOLO_F32, HOLO_F32, HOLO_F32, HOLO_QUAT_F32,
                              HOLO_MODE_CAUSAL,
                              gq, (int64_t)H * m, m, gk, (int64_t)H * m, m,
                              q, (int64_t)H * d, d, k, (int64_t)H * d, d, v, (int64_t)H * d, d,
                              qh, kh, vh_t, P, hol, ws, ws_bytes, NULL);
  if (rc) return die("holo_geom_scan_fwd", holo_last_error());
  rc = holo_attn_fwd(B, T, H, d, HOLO_F32, HOLO_F32, HOLO_QUAT_F32, scale, qh, kh, vh_t, P, o, (int64_t)H * d, d,
                     NULL, NULL);
  if (rc) return die("holo_attn_fwd", holo_last_error());
  rc = holo_attn_masked_fwd(B, T, H, d, HOLO_F32, HOLO_QUAT_F32, HOLO_MODE_CAUSAL, scale, qh, kh, vh_t, P, hol,
                            mask, T, o2, (int64_t)H * d, d, mws, mws_bytes, NULL);
  if (rc) return die("holo_attn_masked_fwd", holo_last_error());
  unsigned* st = dev_alloc(sizeof(unsigned));
  if (!st) return die("hipMalloc", "allocation failed");
  rc = holo_workspace_status(ws, ws_bytes, st, NULL);
  if (rc) return die("holo_workspace_status", holo_last_error());

  /* the bf16 path on the same values rounded to bf16 */
  uint16_t* hb = (uint16_t*)malloc(3 * n_io * 2);
  for (size_t i = 0; i < n_io; ++i) {
    hb[i] = to_bf16(hq[i]);
    hb[n_io + i] = to_bf16(hk[i]);
    hb[2 * n_io + i] = to_bf16(hv[i]);
  }
  uint16_t* qkv16 = dev_alloc(3 * n_io * 2);
  void *qh16 = dev_alloc(n_path * 2), *kh16 = dev_alloc(n_path * 2), *vh16 = dev_alloc(n_path * 2);
  void* P16 = dev_alloc((size_t)B * H * T * nb * 8);
  float* o3 = dev_alloc(n_io * 4);
  if (!qkv16 || !qh16 || !kh16 || !vh16 || !P16 || !o3) return die("hipMalloc", "allocation failed");
  if (hipMemcpy(qkv16, hb, 3 * n_io * 2, hipMemcpyHostToDevice)) return die("hipMemcpy", "upload failed");
  rc = holo_example_core_bf16(B, T, H, d, es, gq, gk, (int64_t)H * m, m, qkv16, qkv16 + n_io, qkv16 + 2 * n_io,
                              (int64_t)H * d, d, qh16, kh16, vh16, P16, ws, ws_bytes, o3, HOLO_F32, NULL);
  if (rc) return die("holo_example_core_bf16", holo_last_error());
  if (hipDeviceSynchronize() != hipSuccess) return die("hipDeviceSynchronize", "kernel error");
  unsigned hst = 1;
  if (hipMemcpy(&hst, st, sizeof(unsigned), hipMemcpyDeviceToHost) || hst != 0)
    return die("workspace status", "the fp32 scan reported a time-out or an overflow");

  float* ho = (float*)malloc(n_io * 4);
  if (hipMemcpy(ho, o, n_io * 4, hipMemcpyDeviceToHost) || write_file(dir, "o_tril.f32", ho, n_io))
    return die("output", "o_tril");
  if (hipMemcpy(ho, o2, n_io * 4, hipMemcpyDeviceToHost) || write_file(dir, "o_ring.f32", ho, n_io))
    return die("output", "o_ring");
  if (hipMemcpy(ho, o3, n_io * 4, hipMemcpyDeviceToHost) || write_file(dir, "o_bf16.f32", ho, n_io))
    return die("output", "o_bf16");
  printf("abi_smoke: ok (B=%d T=%lld H=%d d=%d, ABI %d.%d)\n", B, (long long)T, H, d, holo_abi_version() >> 16,
         holo_abi_version() & 0xffff);
  return 0;
}
