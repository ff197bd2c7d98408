// C ABI of the gfx950 path-ordered attention forward (include/holo_mi355x.h):
// argument validation, status codes and kernel launches. Nothing here
// allocates device memory or synchronises the host.
#include <cmath>
#include <cstdio>
#include <cstdarg>
#include <mutex>
#include <string>

#include "holo_kernels.h"
#include "../../include/holo_mi355x.h"


namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

constexpr int kMaxHeadDim = 96;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// element (b, t, h, c < width) at ptr[(b*T + t)*rs + h*hs + c] must not alias
// across heads/rows in a way the kernels cannot handle: strides positive and
// rows wide enough for all heads.
int check_layout(const char* name, int64_t rs, int64_t hs, int H, int width) {
  if (hs < width || rs < (int64_t)(H - 1) * hs + width)
    return fail(HOLO_ERR_INVALID_ARG, "%s: strides (row %lld, head %lld) too small for %d heads of width %d",
                name, (long long)rs, (long long)hs, H, width);
  return HOLO_OK;
}

int check_common(int B, int64_t T, int H, int d) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0)
    return fail(HOLO_ERR_BAD_SHAPE, "B, T, H, d must be positive (got %d, %lld, %d, %d)",
                B, (long long)T, H, d);
  if (d > kMaxHeadDim)
    return fail(HOLO_ERR_UNSUPPORTED, "head dimension %d above the supported maximum %d", d, kMaxHeadDim);
  if ((int64_t)B * H * ((T + 127) / 128) > 0x7fffffff || T > ((int64_t)1 << 31))
    return fail(HOLO_ERR_UNSUPPORTED, "B*H or T too large");
  return HOLO_OK;
}

// Backward workspace, each region 256-byte aligned: the ticket counter and
// status word, doh, vh and, for fp32
// only, doh_t, qh_t, kh_t (io dtype, B*H*Tp*Dp each; the bf16 kernels read
// the transposed operands from row-major LDS tiles), delta (fp32, B*H*Tp),
// dqh, dkh, dvh (fp32, B*H*Tp*Dp each), the chained suffix sums (fp32,
// B*H*nch*nb*4). Returns the total;
// fills `a` when given.
size_t bwd_layout(int B, int64_t T, int H, int d, size_t es, void* base, holo::BwdArgs* a) {
  const int64_t Tp = holo::padded_seq(T), nch = Tp / holo::kChunk;
  const size_t n = (size_t)B * H * Tp * holo::padded_head_dim(d);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return base ? static_cast<char*>(base) + at : nullptr;
  };
  // ticket counter and status word first (holo_workspace_status reads word 1)
  unsigned* ticket = reinterpret_cast<unsigned*>(take(256));
  void* r[5];
  for (int i = 0; i < 5; ++i) r[i] = (es == 2 && i >= 1 && i <= 3) ? nullptr : take(n * es);
  float* delta = reinterpret_cast<float*>(take((size_t)B * H * Tp * 4));
  float* g[3];
  for (auto& p : g) p = reinterpret_cast<float*>(take(n * 4));
  float* carry = reinterpret_cast<float*>(take((size_t)B * H * nch * (d / 3) * 16));
  if (a) {
    a->doh = r[0]; a->doh_t = r[1]; a->qh_t = r[2]; a->kh_t = r[3]; a->vh = r[4];
    a->delta = delta; a->dqh = g[0]; a->dkh = g[1]; a->dvh = g[2]; a->carry = carry; a->ticket = ticket;
  }
  return off;
}

}  // namespace

extern "C" {

const char* holo_last_error(void) { return g_last_error.c_str(); }

int holo_abi_version(void) { return (6 << 16) | 3; }

int holo_padded_head_dim(int d) { return holo::padded_head_dim(d); }

int64_t holo_padded_seq_len(int64_t T) { return holo::padded_seq(T); }

int holo_qkvg_proj_fwd(int64_t M, int64_t T, int K, int n_qkv, int n_gen,
                       const void* x, int64_t x_rs, const void* w_qkv, const void* w_gq, const void* w_gk,
                       void* qkv, int64_t qkv_rs, float* g, int64_t g_rs, void* stream) {
  g_last_error.clear();
  if (M <= 0 || T <= 0 || K <= 0 || n_qkv < 0 || n_gen < 0 || n_qkv + n_gen == 0)
    return fail(HOLO_ERR_BAD_SHAPE, "M, T, K must be positive, n_qkv, n_gen >= 0, not both 0 (got %lld, %lld, %d, %d, %d)",
                (long long)M, (long long)T, K, n_qkv, n_gen);
  if (M % T != 0) return fail(HOLO_ERR_BAD_SHAPE, "M = %lld is not a whole number of sequences of T = %lld",
                              (long long)M, (long long)T);
  if (K % 64 != 0 || n_qkv % 4 != 0 || n_gen % 4 != 0)
    return fail(HOLO_ERR_UNSUPPORTED, "K = %d must be a multiple of 64 and n_qkv = %d, n_gen = %d multiples of 4",
                K, n_qkv, n_gen);
  if (!x || (n_qkv > 0 && (!w_qkv || !qkv)) || (n_gen > 0 && (!w_gq || !w_gk || !g)))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (!aligned16(x) || (n_qkv > 0 && (!aligned16(w_qkv) || !aligned16(qkv))) ||
      (n_gen > 0 && (!aligned16(w_gq) || !aligned16(w_gk) || !aligned16(g))))
    return fail(HOLO_ERR_INVALID_ARG, "x, weights, qkv and g must be 16-byte aligned");
  if (x_rs < K || x_rs % 8 != 0 || (n_qkv > 0 && (qkv_rs < n_qkv || qkv_rs % 8 != 0)) ||
      (n_gen > 0 && (g_rs < n_gen || g_rs % 4 != 0)))
    return fail(HOLO_ERR_INVALID_ARG, "row strides (x %lld, qkv %lld, g %lld) too small or misaligned",
                (long long)x_rs, (long long)qkv_rs, (long long)g_rs);
  // buffer loads address each operand with 32-bit byte offsets
  if (M * x_rs * 2 > 0x7fffffff || (int64_t)(n_qkv > n_gen ? n_qkv : n_gen) * K * 2 > 0x7fffffff)
    return fail(HOLO_ERR_UNSUPPORTED, "operands above 2 GiB (M = %lld, K = %d)", (long long)M, K);
  holo::QkvgArgs a;
  a.M = M; a.T = T; a.K = K; a.n_qkv = n_qkv; a.n_gen = n_gen;
  a.tm = (int)((M + 255) / 256); a.tnq = (n_qkv + 255) / 256; a.tng = (n_gen + 255) / 256;
  a.x = static_cast<const holo::bf16*>(x); a.ldx = x_rs;
  a.wq = static_cast<const holo::bf16*>(w_qkv);
  a.wg0 = static_cast<const holo::bf16*>(w_gq); a.wg1 = static_cast<const holo::bf16*>(w_gk);
  a.qkv = static_cast<holo::bf16*>(qkv); a.ldq = qkv_rs;
  a.g = g; a.ldg = g_rs;
  const hipError_t e = holo::launch_qkvg(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "projection GEMM launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_edge_hidden_fwd(int64_t M, int64_t T, int K, int n_qkv, int n_hid,
                         const void* x, int64_t x_rs, const void* w_qkv, const void* w1, int64_t w1_rs,
                         const void* b1, void* qkv, int64_t qkv_rs, void* hid, int64_t hid_rs, void* stream) {
  g_last_error.clear();
  if (M <= 0 || T <= 0 || K <= 0 || n_qkv < 0 || n_hid <= 0)
    return fail(HOLO_ERR_BAD_SHAPE, "M, T, K, n_hid must be positive and n_qkv >= 0 (got %lld, %lld, %d, %d, %d)",
                (long long)M, (long long)T, K, n_qkv, n_hid);
  if (M % T != 0) return fail(HOLO_ERR_BAD_SHAPE, "M = %lld is not a whole number of sequences of T = %lld",
                              (long long)M, (long long)T);
  if (K % 64 != 0 || n_qkv % 4 != 0 || n_hid % 4 != 0)
    return fail(HOLO_ERR_UNSUPPORTED, "K = %d must be a multiple of 64 and n_qkv = %d, n_hid = %d multiples of 4",
                K, n_qkv, n_hid);
  if (!x || !w1 || !b1 || !hid || (n_qkv > 0 && (!w_qkv || !qkv)))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (!aligned16(x) || !aligned16(w1) || !aligned16(b1) || !aligned16(hid) ||
      (n_qkv > 0 && (!aligned16(w_qkv) || !aligned16(qkv))))
    return fail(HOLO_ERR_INVALID_ARG, "x, weights, bias, qkv and hid must be 16-byte aligned");
  if (x_rs < K || x_rs % 8 != 0 || w1_rs < 2 * (int64_t)K || w1_rs % 8 != 0 || hid_rs < n_hid || hid_rs % 8 != 0 ||
      (n_qkv > 0 && (qkv_rs < n_qkv || qkv_rs % 8 != 0)))
    return fail(HOLO_ERR_INVALID_ARG, "row strides (x %lld, w1 %lld, qkv %lld, hid %lld) too small or misaligned",
                (long long)x_rs, (long long)w1_rs, (long long)qkv_rs, (long long)hid_rs);
  // 32-bit buffer byte offsets, also for the weight rows of the last
  // 256-feature tile that lie past n_hid (read as zero, never stored)
  const int64_t hid_rows = (n_hid + 255) / 256 * 256;
  if (M * x_rs * 2 > 0x7fffffff || hid_rows * w1_rs * 2 > 0x7fffffff || (int64_t)n_qkv * K * 2 > 0x7fffffff)
    return fail(HOLO_ERR_UNSUPPORTED, "operands above 2 GiB (M = %lld, K = %d, n_hid = %d)", (long long)M, K, n_hid);
  holo::EdgeGemmArgs a{};
  a.M = M; a.T = T; a.K = K; a.n_qkv = n_qkv; a.n_gen = n_hid;
  a.x = static_cast<const holo::bf16*>(x); a.ldx = x_rs;
  a.wq = static_cast<const holo::bf16*>(w_qkv);
  a.wg0 = static_cast<const holo::bf16*>(w1); a.wg1 = a.wg0 + K; a.ldw = w1_rs;
  a.bias = static_cast<const holo::bf16*>(b1);
  a.qkv = static_cast<holo::bf16*>(qkv); a.ldq = qkv_rs;
  a.hid = static_cast<holo::bf16*>(hid); a.ldh = hid_rs;
  const hipError_t e = holo::launch_edge_hidden(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "edge hidden-layer GEMM launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_gemm_f32out_fwd(int64_t M, int K, int N, const void* a_in, int64_t a_rs, const void* w,
                         float* c, int64_t c_rs, void* stream) {
  g_last_error.clear();
  if (M <= 0 || K <= 0 || N <= 0)
    return fail(HOLO_ERR_BAD_SHAPE, "M, K, N must be positive (got %lld, %d, %d)", (long long)M, K, N);
  if (K % 64 != 0 || N % 4 != 0)
    return fail(HOLO_ERR_UNSUPPORTED, "K = %d must be a multiple of 64 and N = %d a multiple of 4", K, N);
  if (!a_in || !w || !c) return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (!aligned16(a_in) || !aligned16(w) || !aligned16(c))
    return fail(HOLO_ERR_INVALID_ARG, "a, w and c must be 16-byte aligned");
  if (a_rs < K || a_rs % 8 != 0 || c_rs < N || c_rs % 4 != 0)
    return fail(HOLO_ERR_INVALID_ARG, "row strides (a %lld, c %lld) too small or misaligned",
                (long long)a_rs, (long long)c_rs);
  const int64_t w_rows = ((int64_t)N + 255) / 256 * 256;
  if (M * a_rs * 2 > 0x7fffffff || w_rows * K * 2 > 0x7fffffff)
    return fail(HOLO_ERR_UNSUPPORTED, "operands above 2 GiB (M = %lld, K = %d, N = %d)", (long long)M, K, N);
  holo::EdgeGemmArgs a{};
  a.M = M; a.T = M; a.K = K; a.n_qkv = 0; a.n_gen = N;
  a.x = static_cast<const holo::bf16*>(a_in); a.ldx = a_rs;
  a.wg0 = static_cast<const holo::bf16*>(w); a.ldw = K;
  a.g = c; a.ldg = c_rs;
  const hipError_t e = holo::launch_gemm_f32out(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "fp32-output GEMM launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

size_t holo_geom_scan_workspace_size(int B, int64_t T, int H, int d) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0) return 0;
  return holo::scan_state_bytes(B, T, H, d);
}

int holo_workspace_status(const void* workspace, size_t workspace_bytes, unsigned* status, void* stream) {
  g_last_error.clear();
  if (!workspace || !status) return fail(HOLO_ERR_INVALID_ARG, "null workspace or status pointer");
  if (workspace_bytes < 8) return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes holds no status word", workspace_bytes);
  const hipError_t e = hipMemcpyAsync(status, static_cast<const unsigned*>(workspace) + 1, sizeof(unsigned),
                                      hipMemcpyDefault, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "status copy: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_geom_scan_fwd(int B, int64_t T, int H, int d,
                       int gen_mode, float edge_scale, int io_dtype, int op_dtype, int gen_dtype,
                       int p_format, int mode,
                       const void* gq, int64_t gq_rs, int64_t gq_hs,
                       const void* gk, int64_t gk_rs, int64_t gk_hs,
                       const void* q, int64_t q_rs, int64_t q_hs,
                       const void* k, int64_t k_rs, int64_t k_hs,
                       const void* v, int64_t v_rs, int64_t v_hs,
                       void* qh, void* kh, void* vh_t, float* P, float* hol,
                       void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  int rc = check_common(B, T, H, d);
  if (rc) return rc;
  if (io_dtype != HOLO_F32 && io_dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "io_dtype %d is not HOLO_F32 or HOLO_BF16", io_dtype);
  if (gen_dtype != HOLO_F32 && gen_dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "gen_dtype %d is not HOLO_F32 or HOLO_BF16", gen_dtype);
  if (io_dtype == HOLO_F32 && gen_dtype != HOLO_F32)
    return fail(HOLO_ERR_UNSUPPORTED, "fp32 keys/values need an fp32 generator");
  if (io_dtype == HOLO_F32 ? op_dtype != HOLO_F32 : (op_dtype != HOLO_BF16 && op_dtype != HOLO_F16))
    return fail(HOLO_ERR_INVALID_ARG, "op_dtype %d with io_dtype %d (fp32 inputs: HOLO_F32; bf16 inputs: "
                "HOLO_BF16 or HOLO_F16)", op_dtype, io_dtype);
  if (gen_mode != HOLO_GEN_ADDITIVE && gen_mode != HOLO_GEN_DIRECT)
    return fail(HOLO_ERR_INVALID_ARG, "gen_mode %d unknown", gen_mode);
  if (p_format != HOLO_QUAT_F32 && p_format != HOLO_QUAT_SNORM16)
    return fail(HOLO_ERR_INVALID_ARG, "p_format %d is not HOLO_QUAT_F32 or HOLO_QUAT_SNORM16", p_format);
  if (mode != HOLO_MODE_CAUSAL && mode != HOLO_MODE_INERT)
    return fail(HOLO_ERR_INVALID_ARG, "mode %d is not HOLO_MODE_CAUSAL or HOLO_MODE_INERT", mode);
  const int nb = d / 3;
  if (!gq || !q || !k || !v || !qh || !kh || !vh_t || (nb > 0 && !P))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (gen_mode == HOLO_GEN_ADDITIVE && !gk)
    return fail(HOLO_ERR_INVALID_ARG, "additive generator needs gk");
  if (gen_mode == HOLO_GEN_DIRECT && gk)
    return fail(HOLO_ERR_INVALID_ARG, "direct generator takes no gk");
  if (nb > 0) {
    if ((rc = check_layout("gq", gq_rs, gq_hs, H, 3 * nb))) return rc;
    // gk row stride 0: one row for every token (a per-head constant)
    if (gk && (rc = check_layout("gk", gk_rs == 0 ? (int64_t)(H - 1) * gk_hs + 3 * nb : gk_rs, gk_hs, H, 3 * nb)))
      return rc;
  }
  if ((rc = check_layout("q", q_rs, q_hs, H, d))) return rc;
  if ((rc = check_layout("k", k_rs, k_hs, H, d))) return rc;
  if ((rc = check_layout("v", v_rs, v_hs, H, d))) return rc;
  if (!aligned16(qh) || !aligned16(kh) || !aligned16(vh_t) || (P && !aligned16(P)) || (hol && !aligned16(hol)))
    return fail(HOLO_ERR_INVALID_ARG, "qh, kh, vh_t, P and hol must be 16-byte aligned");
  size_t need = holo_geom_scan_workspace_size(B, T, H, d);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, workspace ? workspace_bytes : (size_t)0);

  holo::ScanArgs a;
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d);
  a.nbx = (a.Dp + 2) / 3; a.gen_mode = gen_mode;
  a.T = T; a.Tp = holo::padded_seq(T); a.nch = a.Tp / holo::kChunk;
  a.edge_scale = edge_scale;
  a.gq = gq; a.gq_rs = gq_rs; a.gq_hs = gq_hs;
  a.gk = gk; a.gk_rs = gk_rs; a.gk_hs = gk_hs;
  a.q = q; a.q_rs = q_rs; a.q_hs = q_hs;
  a.k = k; a.k_rs = k_rs; a.k_hs = k_hs;
  a.v = v; a.v_rs = v_rs; a.v_hs = v_hs;
  a.qh = qh; a.kh = kh; a.vh_t = vh_t; a.P = P; a.hol = hol;
  a.p_format = p_format;
  a.inert = mode == HOLO_MODE_INERT;
  {
    // 16-byte vector rows: every row start of gq/gk/k/v must be 16-byte aligned
    const size_t ge = gen_dtype == HOLO_F32 ? 4 : 2, ie = io_dtype == HOLO_F32 ? 4 : 2;
    auto al = [](const void* p, int64_t rs, int64_t hs, size_t es) {
      return p == nullptr || (aligned16(p) && (rs * (int64_t)es) % 16 == 0 && (hs * (int64_t)es) % 16 == 0);
    };
    a.wide = (d == 48 || d == 72 || d == 96) && al(gq, gq_rs, gq_hs, ge) && al(gk, gk_rs, gk_hs, ge) &&
             al(q, q_rs, q_hs, ie) && al(k, k_rs, k_hs, ie) && al(v, v_rs, v_hs, ie);
  }
  // chained-scan workspace: the ticket counter and status word (256 bytes),
  // then the chunk products and inclusive prefixes (cleared by the scan's own
  // reset launch)
  a.ticket = static_cast<unsigned*>(workspace);
  a.incl = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  using holo::bf16;
  using holo::f16;
  hipError_t e;
  if (io_dtype == HOLO_F32) e = holo::launch_scan<float, float, float>(a, s);
  else if (op_dtype == HOLO_F16)
    e = gen_dtype == HOLO_F32 ? holo::launch_scan<bf16, f16, float>(a, s) : holo::launch_scan<bf16, f16, bf16>(a, s);
  else
    e = gen_dtype == HOLO_F32 ? holo::launch_scan<bf16, bf16, float>(a, s) : holo::launch_scan<bf16, bf16, bf16>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "scan launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_attn_fwd(int B, int64_t T, int H, int d, int op_dtype, int out_dtype, int p_format, float scale,
                  const void* qh, const void* kh, const void* vh_t, const void* P,
                  void* o, int64_t o_rs, int64_t o_hs, float* lse, void* stream) {
  g_last_error.clear();
  int rc = check_common(B, T, H, d);
  if (rc) return rc;
  if (op_dtype != HOLO_F32 && op_dtype != HOLO_BF16 && op_dtype != HOLO_F16)
    return fail(HOLO_ERR_INVALID_ARG, "op_dtype %d is not HOLO_F32, HOLO_BF16 or HOLO_F16", op_dtype);
  if (out_dtype != HOLO_F32 && !(out_dtype == HOLO_BF16 && op_dtype != HOLO_F32))
    return fail(HOLO_ERR_INVALID_ARG, "out_dtype %d with op_dtype %d (HOLO_F32, or HOLO_BF16 with 16-bit operands)",
                out_dtype, op_dtype);
  const int dtype = op_dtype;
  if (p_format != HOLO_QUAT_F32 && p_format != HOLO_QUAT_SNORM16)
    return fail(HOLO_ERR_INVALID_ARG, "p_format %d is not HOLO_QUAT_F32 or HOLO_QUAT_SNORM16", p_format);
  const int nb = d / 3;
  if (!qh || !kh || !vh_t || !o || (nb > 0 && !P))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if ((rc = check_layout("o", o_rs, o_hs, H, d))) return rc;
  if (!aligned16(qh) || !aligned16(kh) || !aligned16(vh_t) || (P && !aligned16(P)) || (lse && !aligned16(lse)))
    return fail(HOLO_ERR_INVALID_ARG, "qh, kh, vh_t, P and lse must be 16-byte aligned");
  if (!(scale > 0.f) || !(scale < 1e30f))
    return fail(HOLO_ERR_INVALID_ARG, "scale must be positive and finite");
  // key/value tiles of one (b, h) are addressed with 32-bit byte offsets
  if (holo::padded_seq(T) * holo::padded_head_dim(d) * (dtype == HOLO_F32 ? 4 : 2) > 0x7fffffff)
    return fail(HOLO_ERR_UNSUPPORTED, "T = %lld too long for one (b, h) key slice", (long long)T);

  holo::AttnArgs a;
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d);
  a.T = T; a.Tp = holo::padded_seq(T); a.nch = a.Tp / holo::kChunk;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.qh = qh; a.kh = kh; a.vh_t = vh_t; a.P = P;
  a.o = o; a.o_rs = o_rs; a.o_hs = o_hs;
  a.p_format = p_format;
  a.lse = lse;
  hipStream_t s = static_cast<hipStream_t>(stream);
  using holo::bf16;
  using holo::f16;
  const bool of = out_dtype == HOLO_F32;
  hipError_t e = op_dtype == HOLO_F32    ? holo::launch_attn<float, float>(a, s)
                 : op_dtype == HOLO_BF16 ? (of ? holo::launch_attn<bf16, float>(a, s) : holo::launch_attn<bf16, bf16>(a, s))
                                         : (of ? holo::launch_attn<f16, float>(a, s) : holo::launch_attn<f16, bf16>(a, s));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "attention launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

size_t holo_attn_masked_workspace_size(int B, int64_t T, int H, int d, int dtype, int mode, int has_mask) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || (dtype != HOLO_F32 && dtype != HOLO_BF16)) return 0;
  const int64_t Tp = holo::padded_seq(T);
  size_t n = 0;
  if (has_mask)                       // mask bits, then the map of open tiles
    n += (size_t)Tp * (Tp / 64) * 8 + (size_t)((T + 127) / 128) * (Tp / 64);
  return n;
}

}  // extern "C"

namespace {

// Attention dropout's parameters from the drop probability p (0 <= p < 1),
// the 64-bit seed and the counter offset: keep a pair when its Philox word
// is >= round(p 2^32) (ties to even; capped at 2^32 - 1), scale kept weights
// by 1 / (1 - p).
int drop_params(float p, uint64_t seed, uint32_t offset, holo::DropParams& d) {
  if (!(p >= 0.f && p < 1.f)) return fail(HOLO_ERR_INVALID_ARG, "dropout probability %g is not in [0, 1)", (double)p);
  const double t = std::nearbyint((double)p * 4294967296.0);
  d.thr = t >= 4294967295.0 ? 0xffffffffu : (uint32_t)t;
  d.scale = 1.f / (1.f - p);
  d.k0 = (uint32_t)seed;
  d.k1 = (uint32_t)(seed >> 32);
  d.offset = offset;
  return HOLO_OK;
}

// holo_attn_masked_fwd's checks and launch; lse non-null selects the
// training forward (fp32 quaternions, the per-row LSE written), drop
// non-null (with lse) its attention dropout
int masked_fwd(int B, int64_t T, int H, int d, int dtype, int p_format, int mode, float scale,
               const void* qh, const void* kh, const void* vh_t, const void* P, const float* hol,
               const uint8_t* mask, int64_t mask_rs, void* o, int64_t o_rs, int64_t o_hs, float* lse,
               void* workspace, size_t workspace_bytes, void* stream, const holo::DropParams* drop = nullptr) {
  int rc = check_common(B, T, H, d);
  if (rc) return rc;
  if (dtype != HOLO_F32 && dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "dtype %d is not HOLO_F32 or HOLO_BF16", dtype);
  if (p_format != HOLO_QUAT_F32 && p_format != HOLO_QUAT_SNORM16)
    return fail(HOLO_ERR_INVALID_ARG, "p_format %d is not HOLO_QUAT_F32 or HOLO_QUAT_SNORM16", p_format);
  if (mode != HOLO_MODE_CAUSAL && mode != HOLO_MODE_INERT)
    return fail(HOLO_ERR_INVALID_ARG, "mode %d is not HOLO_MODE_CAUSAL or HOLO_MODE_INERT", mode);
  const int nb = d / 3;
  if (!qh || !kh || !vh_t || !o || (nb > 0 && !P))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (mode == HOLO_MODE_CAUSAL && nb > 0 && !hol)
    return fail(HOLO_ERR_INVALID_ARG, "causal mode needs the holonomy (hol)");
  if (mask && mask_rs < T)
    return fail(HOLO_ERR_INVALID_ARG, "mask row stride %lld is below T = %lld", (long long)mask_rs, (long long)T);
  if ((rc = check_layout("o", o_rs, o_hs, H, d))) return rc;
  if (!aligned16(qh) || !aligned16(kh) || !aligned16(vh_t) || (P && !aligned16(P)) || (hol && !aligned16(hol)) ||
      (lse && !aligned16(lse)))
    return fail(HOLO_ERR_INVALID_ARG, "qh, kh, vh_t, P, hol and lse must be 16-byte aligned");
  if (!(scale > 0.f) || !(scale < 1e30f))
    return fail(HOLO_ERR_INVALID_ARG, "scale must be positive and finite");
  const size_t need = holo_attn_masked_workspace_size(B, T, H, d, dtype, mode, mask != nullptr);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, workspace ? workspace_bytes : (size_t)0);

  holo::MaskedLseArgs a;
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d); a.mode = mode;
  a.T = T; a.Tp = holo::padded_seq(T);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.qh = qh; a.kh = kh; a.vh_t = vh_t; a.P = P; a.hol = hol;
  a.mask_bits = nullptr;
  a.tile_act = nullptr;
  a.o = o; a.o_rs = o_rs; a.o_hs = o_hs;
  a.p_format = p_format;
  a.lse = lse;
  a.dropout = drop != nullptr;
  a.drop = drop ? *drop : holo::DropParams{0u, 1.f, 0u, 0u, 0u};
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (mask) {
    a.mask_bits = reinterpret_cast<const uint64_t*>(ws);
    a.tile_act = reinterpret_cast<const uint8_t*>(ws + (size_t)a.Tp * (a.Tp / 64) * 8);
    e = holo::launch_pack_mask(mask, mask_rs, T, a.Tp, reinterpret_cast<uint64_t*>(ws),
                               const_cast<uint8_t*>(a.tile_act), s);
    if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "mask packing launch: %s", hipGetErrorString(e));
  }
  const holo::MaskedArgs& base = a;
  if (lse)
    e = dtype == HOLO_F32 ? holo::launch_attn_masked_lse<float>(a, s) : holo::launch_attn_masked_lse<holo::bf16>(a, s);
  else
    e = dtype == HOLO_F32 ? holo::launch_attn_masked<float>(base, s) : holo::launch_attn_masked<holo::bf16>(base, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "attention launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

}  // namespace

extern "C" {

int holo_attn_masked_fwd(int B, int64_t T, int H, int d, int dtype, int p_format, int mode, float scale,
                         const void* qh, const void* kh, const void* vh_t, const void* P, const float* hol,
                         const uint8_t* mask, int64_t mask_rs,
                         void* o, int64_t o_rs, int64_t o_hs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  return masked_fwd(B, T, H, d, dtype, p_format, mode, scale, qh, kh, vh_t, P, hol, mask, mask_rs, o, o_rs, o_hs,
                    nullptr, workspace, workspace_bytes, stream);
}

int holo_attn_masked_train_fwd(int B, int64_t T, int H, int d, int dtype, int mode, float scale,
                               const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                               const uint8_t* mask, int64_t mask_rs,
                               void* o, int64_t o_rs, int64_t o_hs, float* lse,
                               void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!lse) return fail(HOLO_ERR_INVALID_ARG, "null lse");
  return masked_fwd(B, T, H, d, dtype, HOLO_QUAT_F32, mode, scale, qh, kh, vh_t, P, hol, mask, mask_rs, o, o_rs,
                    o_hs, lse, workspace, workspace_bytes, stream);
}

int holo_attn_masked_dropout_fwd(int B, int64_t T, int H, int d, int dtype, int mode, float scale,
                                 float dropout_p, uint64_t seed, uint32_t offset,
                                 const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                                 const uint8_t* mask, int64_t mask_rs,
                                 void* o, int64_t o_rs, int64_t o_hs, float* lse,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!lse) return fail(HOLO_ERR_INVALID_ARG, "null lse");
  holo::DropParams dp;
  const int rc = drop_params(dropout_p, seed, offset, dp);
  if (rc) return rc;
  return masked_fwd(B, T, H, d, dtype, HOLO_QUAT_F32, mode, scale, qh, kh, vh_t, P, hol, mask, mask_rs, o, o_rs,
                    o_hs, lse, workspace, workspace_bytes, stream, &dp);
}

int holo_dropout_keep_mask(int B, int64_t T, int H, float dropout_p, uint64_t seed, uint32_t offset, uint8_t* keep,
                           void* stream) {
  g_last_error.clear();
  int rc = check_common(B, T, H, 3);
  if (rc) return rc;
  if (!keep) return fail(HOLO_ERR_INVALID_ARG, "null keep");
  holo::DropParams dp;
  if ((rc = drop_params(dropout_p, seed, offset, dp))) return rc;
  const hipError_t e = holo::launch_dropout_keep(B, H, T, dp, keep, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "dropout mask launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

size_t holo_attn_bwd_workspace_size(int B, int64_t T, int H, int d, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || (dtype != HOLO_F32 && dtype != HOLO_BF16)) return 0;
  return bwd_layout(B, T, H, d, dtype == HOLO_F32 ? 4 : 2, nullptr, nullptr);
}

}  // extern "C"

namespace {

// holo_attn_bwd's argument checks; on success every field of `a` but the
// workspace's is set
int bwd_args(int B, int64_t T, int H, int d, int gen_mode, float edge_scale, int io_dtype, int gen_dtype, float scale,
             const void* gq, int64_t gq_rs, int64_t gq_hs, const void* gk, int64_t gk_rs, int64_t gk_hs,
             const void* qh, const void* kh, const void* vh_t, const float* P, const float* lse,
             const void* o, int64_t o_rs, int64_t o_hs, const void* dout, int64_t do_rs, int64_t do_hs,
             void* dq, int64_t dq_rs, int64_t dq_hs, void* dk, int64_t dk_rs, int64_t dk_hs,
             void* dv, int64_t dv_rs, int64_t dv_hs,
             float* dgq, int64_t dgq_rs, int64_t dgq_hs, float* dgk, int64_t dgk_rs, int64_t dgk_hs,
             holo::BwdArgs& a) {
  g_last_error.clear();
  int rc = check_common(B, T, H, d);
  if (rc) return rc;
  if (io_dtype != HOLO_F32 && io_dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "io_dtype %d is not HOLO_F32 or HOLO_BF16", io_dtype);
  if (gen_dtype != HOLO_F32)
    return fail(HOLO_ERR_UNSUPPORTED, "the backward takes an fp32 generator (gen_dtype %d)", gen_dtype);
  if (gen_mode != HOLO_GEN_ADDITIVE && gen_mode != HOLO_GEN_DIRECT)
    return fail(HOLO_ERR_INVALID_ARG, "gen_mode %d unknown", gen_mode);
  const int nb = d / 3;
  if (!qh || !kh || !vh_t || !lse || !o || !dout || !dq || !dk || !dv || (nb > 0 && (!P || !gq || !dgq)))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (nb > 0 && gen_mode == HOLO_GEN_ADDITIVE && (!gk || !dgk))
    return fail(HOLO_ERR_INVALID_ARG, "additive generator needs gk and dgk");
  if (nb > 0) {
    if ((rc = check_layout("gq", gq_rs, gq_hs, H, 3 * nb))) return rc;
    if ((rc = check_layout("dgq", dgq_rs, dgq_hs, H, 3 * nb))) return rc;
    if (gen_mode == HOLO_GEN_ADDITIVE) {
      if ((rc = check_layout("gk", gk_rs, gk_hs, H, 3 * nb))) return rc;
      if ((rc = check_layout("dgk", dgk_rs, dgk_hs, H, 3 * nb))) return rc;
    }
  }
  if ((rc = check_layout("o", o_rs, o_hs, H, d))) return rc;
  if ((rc = check_layout("dout", do_rs, do_hs, H, d))) return rc;
  if ((rc = check_layout("dq", dq_rs, dq_hs, H, d))) return rc;
  if ((rc = check_layout("dk", dk_rs, dk_hs, H, d))) return rc;
  if ((rc = check_layout("dv", dv_rs, dv_hs, H, d))) return rc;
  if (!aligned16(qh) || !aligned16(kh) || !aligned16(vh_t) || (P && !aligned16(P)) || !aligned16(lse))
    return fail(HOLO_ERR_INVALID_ARG, "qh, kh, vh_t, P and lse must be 16-byte aligned");
  if (!(scale > 0.f) || !(scale < 1e30f))
    return fail(HOLO_ERR_INVALID_ARG, "scale must be positive and finite");
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d); a.gen_mode = gen_mode;
  a.T = T; a.Tp = holo::padded_seq(T); a.nch = a.Tp / holo::kChunk;
  a.scale = scale; a.scale_log2 = scale * 1.4426950408889634f; a.edge_scale = edge_scale;
  a.gq = gq; a.gq_rs = gq_rs; a.gq_hs = gq_hs; a.gk = gk; a.gk_rs = gk_rs; a.gk_hs = gk_hs;
  a.qh = qh; a.kh = kh; a.vh_t = vh_t; a.P = P; a.lse = lse;
  a.o = o; a.o_rs = o_rs; a.o_hs = o_hs; a.dout = dout; a.do_rs = do_rs; a.do_hs = do_hs;
  a.dq = dq; a.dq_rs = dq_rs; a.dq_hs = dq_hs; a.dk = dk; a.dk_rs = dk_rs; a.dk_hs = dk_hs;
  a.dv = dv; a.dv_rs = dv_rs; a.dv_hs = dv_hs;
  a.dgq = dgq; a.dgq_rs = dgq_rs; a.dgq_hs = dgq_hs; a.dgk = dgk; a.dgk_rs = dgk_rs; a.dgk_hs = dgk_hs;
  return HOLO_OK;
}

// The exact path's backward workspace: holo_attn_bwd's (bwd_layout), then
// each region 256-byte aligned: the mask bits and the map of open tiles (with
// a mask), and in causal mode qw, dow (io dtype; fp32 also qw_t, dow_t),
// dqw, dkw, dvw (fp32, B*H*Tp*Dp each) and the holonomy's cross sums
// (fp32, B*H*nb*4).
size_t masked_bwd_layout(int B, int64_t T, int H, int d, size_t es, int mode, bool has_mask, void* base,
                         holo::MaskedBwdArgs* a) {
  size_t off = bwd_layout(B, T, H, d, es, base, a);
  const int64_t Tp = holo::padded_seq(T);
  const size_t n = (size_t)B * H * Tp * holo::padded_head_dim(d);
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return base ? static_cast<char*>(base) + at : nullptr;
  };
  char* bits = nullptr;
  char* act = nullptr;
  if (has_mask) {
    bits = take((size_t)Tp * (Tp / 64) * 8);
    act = take((size_t)((T + 127) / 128) * (Tp / 64));
  }
  void* r[4] = {nullptr, nullptr, nullptr, nullptr};
  float* g[4] = {nullptr, nullptr, nullptr, nullptr};
  if (mode == HOLO_MODE_CAUSAL) {
    for (int i = 0; i < 4; ++i) r[i] = (es == 2 && i >= 2) ? nullptr : take(n * es);
    for (int i = 0; i < 3; ++i) g[i] = reinterpret_cast<float*>(take(n * 4));
    g[3] = reinterpret_cast<float*>(take((size_t)B * H * (d / 3) * 16));
  }
  if (a) {
    a->mask_bits = reinterpret_cast<const uint64_t*>(bits);
    a->tile_act = reinterpret_cast<const uint8_t*>(act);
    a->qw = r[0]; a->dow = r[1]; a->qw_t = r[2]; a->dow_t = r[3];
    a->dqw = g[0]; a->dkw = g[1]; a->dvw = g[2]; a->hol_torque = g[3];
  }
  return off;
}

}  // namespace

extern "C" {

int holo_attn_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale, int io_dtype, int gen_dtype,
                  float scale,
                  const void* gq, int64_t gq_rs, int64_t gq_hs, const void* gk, int64_t gk_rs, int64_t gk_hs,
                  const void* qh, const void* kh, const void* vh_t, const float* P, const float* lse,
                  const void* o, int64_t o_rs, int64_t o_hs, const void* dout, int64_t do_rs, int64_t do_hs,
                  void* dq, int64_t dq_rs, int64_t dq_hs, void* dk, int64_t dk_rs, int64_t dk_hs,
                  void* dv, int64_t dv_rs, int64_t dv_hs,
                  float* dgq, int64_t dgq_rs, int64_t dgq_hs, float* dgk, int64_t dgk_rs, int64_t dgk_hs,
                  void* workspace, size_t workspace_bytes, void* stream) {
  holo::BwdArgs a;
  int rc = bwd_args(B, T, H, d, gen_mode, edge_scale, io_dtype, gen_dtype, scale, gq, gq_rs, gq_hs, gk, gk_rs,
                    gk_hs, qh, kh, vh_t, P, lse, o, o_rs, o_hs, dout, do_rs, do_hs, dq, dq_rs, dq_hs, dk, dk_rs,
                    dk_hs, dv, dv_rs, dv_hs, dgq, dgq_rs, dgq_hs, dgk, dgk_rs, dgk_hs, a);
  if (rc) return rc;
  const size_t es = io_dtype == HOLO_F32 ? 4 : 2;
  const size_t need = bwd_layout(B, T, H, d, es, nullptr, nullptr);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, workspace ? workspace_bytes : (size_t)0);
  bwd_layout(B, T, H, d, es, workspace, &a);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = io_dtype == HOLO_F32 ? holo::launch_bwd<float, float>(a, s)
                                      : holo::launch_bwd<holo::bf16, float>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "backward launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

size_t holo_attn_masked_bwd_workspace_size(int B, int64_t T, int H, int d, int dtype, int mode, int has_mask) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || (dtype != HOLO_F32 && dtype != HOLO_BF16) ||
      (mode != HOLO_MODE_CAUSAL && mode != HOLO_MODE_INERT))
    return 0;
  return masked_bwd_layout(B, T, H, d, dtype == HOLO_F32 ? 4 : 2, mode, has_mask != 0, nullptr, nullptr);
}

}  // extern "C"

namespace {

// holo_attn_masked_bwd's checks and launch; drop non-null: the forward's
// attention dropout
int masked_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale, int io_dtype, int gen_dtype,
               int mode, float scale,
                         const void* gq, int64_t gq_rs, int64_t gq_hs, const void* gk, int64_t gk_rs, int64_t gk_hs,
                         const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                         const float* lse, const uint8_t* mask, int64_t mask_rs,
                         const void* o, int64_t o_rs, int64_t o_hs, const void* dout, int64_t do_rs, int64_t do_hs,
                         void* dq, int64_t dq_rs, int64_t dq_hs, void* dk, int64_t dk_rs, int64_t dk_hs,
                         void* dv, int64_t dv_rs, int64_t dv_hs,
                         float* dgq, int64_t dgq_rs, int64_t dgq_hs, float* dgk, int64_t dgk_rs, int64_t dgk_hs,
                         void* workspace, size_t workspace_bytes, void* stream, const holo::DropParams* drop) {
  holo::MaskedBwdArgs a;
  int rc = bwd_args(B, T, H, d, gen_mode, edge_scale, io_dtype, gen_dtype, scale, gq, gq_rs, gq_hs, gk, gk_rs,
                    gk_hs, qh, kh, vh_t, P, lse, o, o_rs, o_hs, dout, do_rs, do_hs, dq, dq_rs, dq_hs, dk, dk_rs,
                    dk_hs, dv, dv_rs, dv_hs, dgq, dgq_rs, dgq_hs, dgk, dgk_rs, dgk_hs, a);
  if (rc) return rc;
  if (mode != HOLO_MODE_CAUSAL && mode != HOLO_MODE_INERT)
    return fail(HOLO_ERR_INVALID_ARG, "mode %d is not HOLO_MODE_CAUSAL or HOLO_MODE_INERT", mode);
  if (mode == HOLO_MODE_CAUSAL && a.nb > 0 && (!hol || !aligned16(hol)))
    return fail(HOLO_ERR_INVALID_ARG, "causal mode needs the holonomy (hol, 16-byte aligned)");
  if (mask && mask_rs < T)
    return fail(HOLO_ERR_INVALID_ARG, "mask row stride %lld is below T = %lld", (long long)mask_rs, (long long)T);
  const size_t es = io_dtype == HOLO_F32 ? 4 : 2;
  const size_t need = masked_bwd_layout(B, T, H, d, es, mode, mask != nullptr, nullptr, nullptr);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, workspace ? workspace_bytes : (size_t)0);
  masked_bwd_layout(B, T, H, d, es, mode, mask != nullptr, workspace, &a);
  a.mode = mode == HOLO_MODE_CAUSAL ? 0 : 1;
  a.hol = hol;
  a.dropout = drop != nullptr;
  a.drop = drop ? *drop : holo::DropParams{0u, 1.f, 0u, 0u, 0u};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (mask) {
    e = holo::launch_pack_mask(mask, mask_rs, T, a.Tp, const_cast<uint64_t*>(a.mask_bits),
                               const_cast<uint8_t*>(a.tile_act), s);
    if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "mask packing launch: %s", hipGetErrorString(e));
  }
  e = io_dtype == HOLO_F32 ? holo::launch_masked_bwd<float, float>(a, s)
                           : holo::launch_masked_bwd<holo::bf16, float>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "backward launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

}  // namespace

extern "C" {

int holo_attn_masked_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale, int io_dtype, int gen_dtype,
                         int mode, float scale,
                         const void* gq, int64_t gq_rs, int64_t gq_hs, const void* gk, int64_t gk_rs, int64_t gk_hs,
                         const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                         const float* lse, const uint8_t* mask, int64_t mask_rs,
                         const void* o, int64_t o_rs, int64_t o_hs, const void* dout, int64_t do_rs, int64_t do_hs,
                         void* dq, int64_t dq_rs, int64_t dq_hs, void* dk, int64_t dk_rs, int64_t dk_hs,
                         void* dv, int64_t dv_rs, int64_t dv_hs,
                         float* dgq, int64_t dgq_rs, int64_t dgq_hs, float* dgk, int64_t dgk_rs, int64_t dgk_hs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return masked_bwd(B, T, H, d, gen_mode, edge_scale, io_dtype, gen_dtype, mode, scale, gq, gq_rs, gq_hs, gk, gk_rs,
                    gk_hs, qh, kh, vh_t, P, hol, lse, mask, mask_rs, o, o_rs, o_hs, dout, do_rs, do_hs, dq, dq_rs,
                    dq_hs, dk, dk_rs, dk_hs, dv, dv_rs, dv_hs, dgq, dgq_rs, dgq_hs, dgk, dgk_rs, dgk_hs, workspace,
                    workspace_bytes, stream, nullptr);
}

int holo_attn_masked_dropout_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale, int io_dtype,
                                 int gen_dtype, int mode, float scale, float dropout_p, uint64_t seed, uint32_t offset,
                                 const void* gq, int64_t gq_rs, int64_t gq_hs, const void* gk, int64_t gk_rs,
                                 int64_t gk_hs, const void* qh, const void* kh, const void* vh_t, const float* P,
                                 const float* hol, const float* lse, const uint8_t* mask, int64_t mask_rs,
                                 const void* o, int64_t o_rs, int64_t o_hs, const void* dout, int64_t do_rs,
                                 int64_t do_hs, void* dq, int64_t dq_rs, int64_t dq_hs, void* dk, int64_t dk_rs,
                                 int64_t dk_hs, void* dv, int64_t dv_rs, int64_t dv_hs,
                                 float* dgq, int64_t dgq_rs, int64_t dgq_hs, float* dgk, int64_t dgk_rs,
                                 int64_t dgk_hs, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  holo::DropParams dp;
  const int rc = drop_params(dropout_p, seed, offset, dp);
  if (rc) return rc;
  return masked_bwd(B, T, H, d, gen_mode, edge_scale, io_dtype, gen_dtype, mode, scale, gq, gq_rs, gq_hs, gk, gk_rs,
                    gk_hs, qh, kh, vh_t, P, hol, lse, mask, mask_rs, o, o_rs, o_hs, dout, do_rs, do_hs, dq, dq_rs,
                    dq_hs, dk, dk_rs, dk_hs, dv, dv_rs, dv_hs, dgq, dgq_rs, dgq_hs, dgk, dgk_rs, dgk_hs, workspace,
                    workspace_bytes, stream, &dp);
}

int holo_add_layernorm_fwd(int64_t n, int d, int dtype, float eps, const void* x, int64_t x_rs,
                           const void* delta, int64_t delta_rs, const void* weight, const void* bias,
                           void* h, int64_t h_rs, void* y, int64_t y_rs, void* stream) {
  g_last_error.clear();
  if (n < 0 || d <= 0) return fail(HOLO_ERR_BAD_SHAPE, "n must be >= 0 and d > 0");
  if (dtype != HOLO_F32 && dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "dtype %d is not HOLO_F32 or HOLO_BF16", dtype);
  const int64_t e16 = dtype == HOLO_F32 ? 4 : 8;       // elements per 16 bytes
  if (d % e16 || d > 1024 * e16)
    return fail(HOLO_ERR_UNSUPPORTED, "d = %d: must be a multiple of %d and at most %d for this dtype", d,
                (int)e16, (int)(1024 * e16));
  if (!(eps > 0.f)) return fail(HOLO_ERR_INVALID_ARG, "eps must be positive");
  if (n == 0) return HOLO_OK;
  if (!x || !delta || !weight || !bias || !h || !y) return fail(HOLO_ERR_INVALID_ARG, "null pointer");
  for (const int64_t rs : {x_rs, delta_rs, h_rs, y_rs})
    if (rs < d || rs % e16) return fail(HOLO_ERR_INVALID_ARG, "row strides must be >= d and 16-byte multiples");
  if (!aligned16(x) || !aligned16(delta) || !aligned16(weight) || !aligned16(bias) || !aligned16(h) || !aligned16(y))
    return fail(HOLO_ERR_INVALID_ARG, "pointers must be 16-byte aligned");
  holo::AddNormArgs a;
  a.n = n; a.d = d; a.eps = eps;
  a.x = x; a.x_rs = x_rs; a.delta = delta; a.delta_rs = delta_rs; a.w = weight; a.b = bias;
  a.h = h; a.h_rs = h_rs; a.y = y; a.y_rs = y_rs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == HOLO_F32 ? holo::launch_add_layernorm<float>(a, s)
                                   : holo::launch_add_layernorm<holo::bf16>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "add_layernorm launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_quat_to_dense(int64_t n, int d, const float* quat, float* dense, void* stream) {
  g_last_error.clear();
  if (n < 0 || d <= 0) return fail(HOLO_ERR_BAD_SHAPE, "n must be >= 0 and d > 0");
  if (n > 0 && ((d >= 3 && !quat) || !dense)) return fail(HOLO_ERR_INVALID_ARG, "null pointer");
  if (quat && !aligned16(quat)) return fail(HOLO_ERR_INVALID_ARG, "quat must be 16-byte aligned");
  hipError_t e = holo::launch_quat_to_dense(n, d, quat, dense, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "quat_to_dense launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

int holo_decode_geom_fwd(int B, int H, int d, int64_t t, int64_t capacity,
                         int gen_mode, float edge_scale, int io_dtype, int gen_dtype,
                         const void* gq, int64_t gq_bs, int64_t gq_hs,
                         const void* gk, int64_t gk_bs, int64_t gk_hs,
                         const void* q, int64_t q_bs, int64_t q_hs,
                         const void* k, int64_t k_bs, int64_t k_hs,
                         const void* v, int64_t v_bs, int64_t v_hs,
                         float* P, void* qh, void* kh_cache, void* vh_cache, void* stream) {
  g_last_error.clear();
  int rc = check_common(B, capacity, H, d);
  if (rc) return rc;
  if (t < 0 || capacity % holo::kChunk != 0 || t >= capacity)
    return fail(HOLO_ERR_BAD_SHAPE, "need 0 <= t < capacity and capacity a multiple of 64 (t=%lld, capacity=%lld)",
                (long long)t, (long long)capacity);
  if (io_dtype != HOLO_F32 && io_dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "io_dtype %d is not HOLO_F32 or HOLO_BF16", io_dtype);
  if (gen_dtype != HOLO_F32 && gen_dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "gen_dtype %d is not HOLO_F32 or HOLO_BF16", gen_dtype);
  if (io_dtype == HOLO_F32 && gen_dtype != HOLO_F32)
    return fail(HOLO_ERR_UNSUPPORTED, "fp32 keys/values need an fp32 generator");
  if (gen_mode != HOLO_GEN_ADDITIVE && gen_mode != HOLO_GEN_DIRECT)
    return fail(HOLO_ERR_INVALID_ARG, "gen_mode %d unknown", gen_mode);
  const int nb = d / 3;
  if (!q || !k || !v || !qh || !kh_cache || !vh_cache || (nb > 0 && !P))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (t > 0 && nb > 0 && (!gq || (gen_mode == HOLO_GEN_ADDITIVE) != (gk != nullptr)))
    return fail(HOLO_ERR_INVALID_ARG, "link parameters: gq (and gk in additive mode only) are required for t > 0");
  if (!aligned16(qh) || !aligned16(kh_cache) || !aligned16(vh_cache) || (P && !aligned16(P)))
    return fail(HOLO_ERR_INVALID_ARG, "qh, the caches and P must be 16-byte aligned");

  holo::DecodeGeomArgs a;
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d); a.gen_mode = gen_mode;
  a.t = t; a.cap = capacity; a.edge_scale = edge_scale;
  a.gq = gq; a.gq_bs = gq_bs; a.gq_hs = gq_hs;
  a.gk = gk; a.gk_bs = gk_bs; a.gk_hs = gk_hs;
  a.q = q; a.q_bs = q_bs; a.q_hs = q_hs;
  a.k = k; a.k_bs = k_bs; a.k_hs = k_hs;
  a.v = v; a.v_bs = v_bs; a.v_hs = v_hs;
  a.P = P; a.qh = qh; a.kc = kh_cache; a.vc = vh_cache;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = io_dtype == HOLO_F32 ? holo::launch_decode_geom<float, float>(a, s)
                 : gen_dtype == HOLO_F32 ? holo::launch_decode_geom<holo::bf16, float>(a, s)
                                         : holo::launch_decode_geom<holo::bf16, holo::bf16>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "decode geometry launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

size_t holo_decode_attn_workspace_size(int B, int H, int d, int64_t t) {
  if (B <= 0 || H <= 0 || d <= 0 || t < 0) return 0;
  return (size_t)B * H * holo::decode_splits(t) * (holo::padded_head_dim(d) + 2) * sizeof(float);
}

int holo_decode_attn_fwd(int B, int H, int d, int64_t t, int64_t capacity, int dtype, float scale,
                         const void* qh, const void* kh_cache, const void* vh_cache, const float* P,
                         void* o, int64_t o_bs, int64_t o_hs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  int rc = check_common(B, capacity, H, d);
  if (rc) return rc;
  if (t < 0 || capacity % holo::kChunk != 0 || t >= capacity)
    return fail(HOLO_ERR_BAD_SHAPE, "need 0 <= t < capacity and capacity a multiple of 64 (t=%lld, capacity=%lld)",
                (long long)t, (long long)capacity);
  if (dtype != HOLO_F32 && dtype != HOLO_BF16)
    return fail(HOLO_ERR_INVALID_ARG, "dtype %d is not HOLO_F32 or HOLO_BF16", dtype);
  if (!(scale > 0.f) || !(scale < 1e30f))
    return fail(HOLO_ERR_INVALID_ARG, "scale must be positive and finite");
  const int nb = d / 3;
  if (!qh || !kh_cache || !vh_cache || !o || (nb > 0 && !P))
    return fail(HOLO_ERR_INVALID_ARG, "null input or output pointer");
  if (o_hs < d || o_bs < (int64_t)H * o_hs)
    return fail(HOLO_ERR_INVALID_ARG, "o strides (batch %lld, head %lld) overlap", (long long)o_bs, (long long)o_hs);
  if (!aligned16(qh) || !aligned16(kh_cache) || !aligned16(vh_cache) || (P && !aligned16(P)))
    return fail(HOLO_ERR_INVALID_ARG, "qh, the caches and P must be 16-byte aligned");
  if (capacity * holo::padded_head_dim(d) * (dtype == HOLO_F32 ? 4 : 2) > 0x7fffffff)
    return fail(HOLO_ERR_UNSUPPORTED, "capacity %lld too long for one (b, h) key slice", (long long)capacity);
  const size_t need = holo_decode_attn_workspace_size(B, H, d, t);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(HOLO_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, workspace ? workspace_bytes : (size_t)0);

  holo::DecodeAttnArgs a;
  a.B = B; a.H = H; a.d = d; a.nb = nb; a.Dp = holo::padded_head_dim(d);
  a.t = t; a.cap = capacity; a.nsplit = holo::decode_splits(t);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.qh = qh; a.kc = kh_cache; a.vc = vh_cache; a.P = P;
  a.o = o; a.o_bs = o_bs; a.o_hs = o_hs;
  a.ws = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == HOLO_F32 ? holo::launch_decode_attn<float>(a, s)
                                   : holo::launch_decode_attn<holo::bf16>(a, s);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "decode attention launch: %s", hipGetErrorString(e));
  return HOLO_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// holo_geom_scan_fwd_static: the scan with its chained state in a static
// device array instead of a caller workspace, for callers that cannot
// allocate (graph capture, serving loops). One array per device, held until
// the process ends; every call on a device shares it, so calls that overlap
// in time on one device race. The scan's own reset kernel clears the state
// and the ticket counter at the start of every call.
namespace {

constexpr size_t kScratchBytes = HOLO_SCAN_STATIC_SCRATCH_BYTES;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];   // device address of `scratch`, per device

// Device address of the current device's `scratch` (the host-side symbol is
// only a stand-in for it), resolved once per device with that device current.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HOLO_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kScratchDevices)
    return fail(HOLO_ERR_UNSUPPORTED, "device %d beyond the %d devices the static scratch tracks", dev,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(HOLO_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HOLO_OK;
}

}  // namespace

extern "C" int holo_geom_scan_fwd_static(int B, int64_t T, int H, int d,
                                         int gen_mode, float edge_scale, int io_dtype, int op_dtype, int gen_dtype,
                                         int p_format, int mode,
                                         const void* gq, int64_t gq_rs, int64_t gq_hs,
                                         const void* gk, int64_t gk_rs, int64_t gk_hs,
                                         const void* q, int64_t q_rs, int64_t q_hs,
                                         const void* k, int64_t k_rs, int64_t k_hs,
                                         const void* v, int64_t v_rs, int64_t v_hs,
                                         void* qh, void* kh, void* vh_t, float* P, float* hol, void* stream) {
  g_last_error.clear();
  const size_t need = holo_geom_scan_workspace_size(B, T, H, d);
  if (need > kScratchBytes)
    return fail(HOLO_ERR_UNSUPPORTED,
                "B=%d T=%lld H=%d d=%d needs %zu bytes of chained scan state, above the %zu-byte static scratch "
                "(holo_geom_scan_fwd takes a caller workspace of any size)",
                B, (long long)T, H, d, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return holo_geom_scan_fwd(B, T, H, d, gen_mode, edge_scale, io_dtype, op_dtype, gen_dtype, p_format, mode,
                            gq, gq_rs, gq_hs, gk, gk_rs, gk_hs, q, q_rs, q_hs, k, k_rs, k_hs, v, v_rs, v_hs,
                            qh, kh, vh_t, P, hol, ws, kScratchBytes, stream);
}
