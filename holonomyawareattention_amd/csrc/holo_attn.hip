// Causal path-ordered attention forward on gfx950 MFMA.
//
// Reference behaviour (core/attention_fast_chunked.py:105-171 with a tril mask;
// kernel/attention_kernel.py:40-116 is the Triton form of the same math):
//   qh_i = P_i^T q_i
//   oh_i = sum_{j<=i} softmax_j(scale * qh_i . kh_j) vh_j      (online softmax)
//   o_i  = P_i oh_i
// The wrap branch (i < j) of the reference is always masked under tril and is
// not computed.
//
// Work decomposition: one workgroup (4 waves) per (b, h, 128-query tile); each
// wave owns 32 queries. Key/value tiles of 64 keys are staged in LDS
// (kh row-major, vh already stored transposed by the scan), and each wave
// computes
//     S^T (64 keys x 32 queries) = K (64 x Dp) . Q^T (Dp x 32)
//     O^T (Dp x 32 queries)     += V^T (Dp x 64) . P^T (64 x 32)
// on 32x32 MFMA tiles. With keys on the MFMA rows and queries on the lanes,
// a lane holds 32 of a query's 64 scores in registers and its partner lane
// (l ^ 32) the other 32: the row max and the rescale of the accumulator are
// per-lane operations plus one cross-lane exchange, and the exponentiated
// scores are already in the register layout of the P^T operand.
// The query transport (prologue) and the back-rotation (epilogue) are fused:
// the workgroup stages its 128 query rows through LDS, rotating each 3-dim
// block by its stored quaternion.
#include <type_traits>

#include "holo_kernels.h"

namespace holo {

constexpr int kBM = 128;                  // queries per workgroup
constexpr int kBN = 64;                   // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <typename T, int DP> struct AttnCfg {
  static constexpr int E = 16 / sizeof(T);             // elements per 16 B
  static constexpr int KS = DP + E;                     // padded LDS row strides
  static constexpr int VS = kBN + E;
  static constexpr int QS = DP + E;
  static constexpr int OS = DP + 4;                     // fp32 staging
  static constexpr int NBX = (DP + 2) / 3;              // 3-dim groups covering DP
  static constexpr size_t kv_bytes = (size_t)(kBN * KS + DP * VS) * sizeof(T);
  static constexpr size_t q_bytes = (size_t)kBM * QS * sizeof(T);
  static constexpr size_t o_bytes = (size_t)kBM * OS * sizeof(float);
  static constexpr size_t lds = kv_bytes > q_bytes ? (kv_bytes > o_bytes ? kv_bytes : o_bytes)
                                                   : (q_bytes > o_bytes ? q_bytes : o_bytes);
};

template <typename T, int DP>
__global__ void __launch_bounds__(kThreads) attn_fwd(AttnArgs a) {
  using C = AttnCfg<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  T* Ks = reinterpret_cast<T*>(smem);
  T* Vs = Ks + kBN * C::KS;
  T* Qs = reinterpret_cast<T*>(smem);
  float* Os = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int lr = lane & 31;               // query column of this lane (MFMA col)
  const int g = lane >> 5;                // lane half
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int64_t ntile = (a.T + kBM - 1) / kBM;
  const int64_t q0 = (ntile - 1 - blockIdx.y) * kBM;   // longest tiles first
  const int64_t qw = q0 + 32 * w;                       // first query of this wave
  const int64_t qi = qw + lr;                           // this lane's query

  // ---- prologue: qh = P^T q for the tile's rows, staged in LDS ----
  for (int idx = tid; idx < kBM * C::NBX; idx += kThreads) {
    int r = idx / C::NBX, blk = idx % C::NBX, c0 = 3 * blk;
    int64_t t = q0 + r;
    float u[3] = {0.f, 0.f, 0.f};
    if (t < a.T) {
      const T* qr = reinterpret_cast<const T*>(a.q) + (b * a.T + t) * a.q_rs + h * a.q_hs + c0;
      for (int j = 0; j < 3; ++j)
        if (c0 + j < a.d) u[j] = to_f32(qr[j]);
      if (blk < a.nb) {
        rot3 R = qmat(load_quat(a.P + ((bh * a.T + t) * a.nb + blk) * 4));
        float y0, y1, y2;
        rot_t_apply(R, u[0], u[1], u[2], y0, y1, y2);
        u[0] = y0; u[1] = y1; u[2] = y2;
      }
    }
    for (int j = 0; j < 3; ++j)
      if (c0 + j < DP) Qs[r * C::QS + c0 + j] = from_f32<T>(u[j]);
  }
  __syncthreads();

  constexpr bool kBF = sizeof(T) == 2;
  constexpr int QF = kBF ? DP / 16 : DP / 2;            // Q^T operand steps
  typedef typename std::conditional<kBF, bf16x8, float>::type qfrag_t;
  qfrag_t qf[QF];
  for (int s = 0; s < QF; ++s) {
    if constexpr (kBF) qf[s] = *reinterpret_cast<const bf16x8*>(&Qs[(32 * w + lr) * C::QS + 16 * s + 8 * g]);
    else qf[s] = Qs[(32 * w + lr) * C::QS + 2 * s + g];
  }
  __syncthreads();

  f32x16 O[DP / 32];
  for (int i = 0; i < DP / 32; ++i) O[i] = f32x16{};
  float m_run = -1e30f, l_run = 0.f;

  int64_t kend = q0 + kBM; if (kend > a.T) kend = a.T;
  const int nkv = (int)((kend + kBN - 1) / kBN);
  const T* kbase = reinterpret_cast<const T*>(a.kh) + (int64_t)bh * a.Tp * DP;
  const T* vbase = reinterpret_cast<const T*>(a.vh_t) + (int64_t)bh * a.nch * DP * kBN;

  for (int kt = 0; kt < nkv; ++kt) {
    const int64_t k0 = (int64_t)kt * kBN;
    // ---- stage the key tile (row-major) and the value tile (transposed) ----
    {
      constexpr int RC = DP / C::E;                    // 16 B chunks per key row
      const uint4* ksrc = reinterpret_cast<const uint4*>(kbase + k0 * DP);
      for (int i = tid; i < kBN * RC; i += kThreads) {
        int r = i / RC, cc = i % RC;
        *reinterpret_cast<uint4*>(&Ks[r * C::KS + cc * C::E]) = ksrc[i];
      }
      constexpr int VC = kBN / C::E;                   // 16 B chunks per value row
      const uint4* vsrc = reinterpret_cast<const uint4*>(vbase + (int64_t)kt * DP * kBN);
      for (int i = tid; i < DP * VC; i += kThreads) {
        int r = i / VC, cc = i % VC;
        *reinterpret_cast<uint4*>(&Vs[r * C::VS + cc * C::E]) = vsrc[i];
      }
    }
    __syncthreads();

    if (qw + 31 >= k0 && qw < a.T) {
      // ---- S^T = K Q^T ----
      f32x16 S[2] = {f32x16{}, f32x16{}};
      for (int kb = 0; kb < 2; ++kb) {
        for (int s = 0; s < QF; ++s) {
          if constexpr (kBF) {
            bf16x8 av = *reinterpret_cast<const bf16x8*>(&Ks[(32 * kb + lr) * C::KS + 16 * s + 8 * g]);
            S[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qf[s], S[kb], 0, 0, 0);
          } else {
            float av = Ks[(32 * kb + lr) * C::KS + 2 * s + g];
            S[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, qf[s], S[kb], 0, 0, 0);
          }
        }
      }
      // ---- online softmax (log2 domain), per lane = per query ----
      const bool need_mask = (k0 + kBN - 1 > qw);
      float mx = -INFINITY;
      for (int kb = 0; kb < 2; ++kb)
        for (int r = 0; r < 16; ++r) {
          float s = S[kb][r] * a.scale_log2;
          if (need_mask) {
            int64_t key = k0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key > qi) s = -INFINITY;
          }
          S[kb][r] = s;
          mx = fmaxf(mx, s);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float corr = exp2f(m_run - m_new);
      m_run = m_new;
      float ls = 0.f;
      for (int kb = 0; kb < 2; ++kb)
        for (int r = 0; r < 16; ++r) {
          float p = exp2f(S[kb][r] - m_new);
          S[kb][r] = p;
          ls += p;
        }
      l_run = l_run * corr + ls;
      for (int i = 0; i < DP / 32; ++i)
        for (int r = 0; r < 16; ++r) O[i][r] *= corr;

      // ---- O^T += V^T P^T ----
      if constexpr (kBF) {
        bf16x8 pb[2][2];
        for (int kb = 0; kb < 2; ++kb)
          for (int hh = 0; hh < 2; ++hh)
            for (int e = 0; e < 8; ++e) pb[kb][hh][e] = (bf16)S[kb][8 * hh + e];
        for (int db = 0; db < DP / 32; ++db)
          for (int kb = 0; kb < 2; ++kb)
            for (int hh = 0; hh < 2; ++hh) {
              const T* vr = &Vs[(32 * db + lr) * C::VS + 32 * kb + 16 * hh + 4 * g];
              bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
              bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
              bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
              O[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[kb][hh], O[db], 0, 0, 0);
            }
      } else {
        for (int db = 0; db < DP / 32; ++db)
          for (int kb = 0; kb < 2; ++kb)
            for (int r = 0; r < 16; ++r) {
              float av = Vs[(32 * db + lr) * C::VS + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3)];
              O[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, S[kb][r], O[db], 0, 0, 0);
            }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise, stage O^T, back-rotate o = P oh, store ----
  float lt = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.f / fmaxf(lt, 1e-20f);
  for (int db = 0; db < DP / 32; ++db)
    for (int r = 0; r < 16; ++r)
      Os[(32 * w + lr) * C::OS + 32 * db + 8 * (r >> 2) + 4 * g + (r & 3)] = O[db][r] * inv;
  __syncthreads();
  for (int idx = tid; idx < kBM * C::NBX; idx += kThreads) {
    int r = idx / C::NBX, blk = idx % C::NBX, c0 = 3 * blk;
    int64_t t = q0 + r;
    if (t >= a.T || c0 >= a.d) continue;
    float u[3];
    for (int j = 0; j < 3; ++j) u[j] = (c0 + j < DP) ? Os[r * C::OS + c0 + j] : 0.f;
    if (blk < a.nb) {
      rot3 R = qmat(load_quat(a.P + ((bh * a.T + t) * a.nb + blk) * 4));
      float y0, y1, y2;
      rot_apply(R, u[0], u[1], u[2], y0, y1, y2);
      u[0] = y0; u[1] = y1; u[2] = y2;
    }
    T* orow = reinterpret_cast<T*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs + c0;
    for (int j = 0; j < 3; ++j)
      if (c0 + j < a.d) orow[j] = from_f32<T>(u[j]);
  }
}

template <typename T, int DP>
static hipError_t launch_attn_dp(const AttnArgs& a, hipStream_t s) {
  using C = AttnCfg<T, DP>;
  const int64_t ntile = (a.T + kBM - 1) / kBM;
  hipLaunchKernelGGL((attn_fwd<T, DP>), dim3(a.B * a.H, (unsigned)ntile), dim3(kThreads),
                     C::lds, s, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_attn(const AttnArgs& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_attn_dp<T, 32>(a, s);
    case 64: return launch_attn_dp<T, 64>(a, s);
    case 96: return launch_attn_dp<T, 96>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t launch_attn<float>(const AttnArgs&, hipStream_t);
template hipError_t launch_attn<bf16>(const AttnArgs&, hipStream_t);

// ---- quaternion -> dense rotation matrices (geometry output) ----
__global__ void __launch_bounds__(256) quat_to_dense(int64_t n, int d, int nb, const float* q, float* out) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = n * d * d;
  if (gid >= total) return;
  int64_t i = gid / ((int64_t)d * d);
  int r = (gid / d) % d, c = gid % d;
  float val = 0.f;
  int br = r / 3, bc = c / 3;
  if (br < nb && bc < nb) {
    if (br == bc) {
      rot3 R = qmat(load_quat(q + (i * nb + br) * 4));
      val = R.m[r - 3 * br][c - 3 * bc];
    }
  } else if (r == c) {
    val = 1.f;
  }
  out[gid] = val;
}

hipError_t launch_quat_to_dense(int64_t n, int d, const float* q, float* out, hipStream_t s) {
  int64_t total = n * d * d;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(quat_to_dense, dim3((total + 255) / 256), dim3(256), 0, s, n, d, d / 3, q, out);
  return hipGetLastError();
}

}  // namespace holo
