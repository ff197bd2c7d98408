// Incremental decode of the path-ordered attention forward (gfx950).
//
// After a prefill of tokens 0..t-1, one new token t per (b, h) and step:
//   a_{t-1} = edge_scale * (gq_{t-1} + gk_t)   additive  (core/attention_fast_chunked.py:80-84)
//   a_{t-1} = edge_scale * g_{t-1}             direct    (:73-79, g from the edge MLP of (x_{t-1}, x_t))
//   P_t     = exp(skew(a_{t-1})) P_{t-1}                 (:86-94)
//   qh_t = P_t^T q_t, kh_t = P_t^T k_t, vh_t = P_t^T v_t  (:108-110)
//   o_t  = P_t sum_{j<=t} softmax_j(scale * qh_t . kh_j) vh_j   (row t of :119-171)
// Row t of the full-sequence forward is exactly this: the edge t-1 -> t uses
// only x_{t-1} and x_t, and the closing edge only enters the holonomy.
//
// Keys and values stay in the frame of token 0 (the global frame), so the
// cache never needs re-rotation; it uses the scan's own layouts with a
// capacity in place of the padded length: kh (B, H, cap, Dp) row-major and
// vh (B, H, cap/64, Dp, 64) in transposed 64-key tiles.
//
// Kernels:
//   decode_geom        one workgroup per (b, h): compose the new link into the
//                      running P (fp32 quaternions), transport q, k, v, write
//                      qh and append row t to the caches;
//   decode_attn_split  one workgroup per (b, h, 256-key segment): scores by
//                      v_dot2 over the key rows, segment max / sum, and the
//                      segment's P V from the transposed value tiles read as
//                      contiguous 16-byte lanes; writes (max, sum, o) partials;
//   decode_attn_combine one workgroup per (b, h): merges the segments and
//                      back-rotates o by P_t.
// Each step reads every cached key and value once: the kernels are HBM bound.
#include "holo_kernels.h"

namespace holo {

constexpr int kDecodeSplit = 256;          // keys per decode_attn_split workgroup

template <typename IO, typename GT>
__global__ void __launch_bounds__(64) decode_geom(DecodeGeomArgs a) {
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int j = threadIdx.x;
  const int nb = a.nb;
  const IO* q = reinterpret_cast<const IO*>(a.q) + (int64_t)b * a.q_bs + (int64_t)h * a.q_hs;
  const IO* k = reinterpret_cast<const IO*>(a.k) + (int64_t)b * a.k_bs + (int64_t)h * a.k_hs;
  const IO* v = reinterpret_cast<const IO*>(a.v) + (int64_t)b * a.v_bs + (int64_t)h * a.v_hs;
  IO* qh = reinterpret_cast<IO*>(a.qh) + (int64_t)bh * a.Dp;
  IO* krow = reinterpret_cast<IO*>(a.kc) + ((int64_t)bh * a.cap + a.t) * a.Dp;
  // element c of the new value column sits at vcol[c * kChunk]
  IO* vcol = reinterpret_cast<IO*>(a.vc) + ((int64_t)bh * (a.cap / kChunk) + a.t / kChunk) * a.Dp * kChunk +
             a.t % kChunk;
  if (j < nb) {
    float* ps = a.P + ((int64_t)bh * nb + j) * 4;
    quat P = load_quat(ps);
    if (a.t > 0) {
      const GT* gq = reinterpret_cast<const GT*>(a.gq) + (int64_t)b * a.gq_bs + (int64_t)h * a.gq_hs + 3 * j;
      float p0 = to_f32(gq[0]), p1 = to_f32(gq[1]), p2 = to_f32(gq[2]);
      if (a.gen_mode == 0) {
        const GT* gk = reinterpret_cast<const GT*>(a.gk) + (int64_t)b * a.gk_bs + (int64_t)h * a.gk_hs + 3 * j;
        p0 += to_f32(gk[0]); p1 += to_f32(gk[1]); p2 += to_f32(gk[2]);
      }
      const float es = a.edge_scale;
      P = qmul(qexp_skew(p0 * es, p1 * es, p2 * es), P);
      store_quat(ps, P);
    }
    const rot3 R = qmat(P);
    const int c = 3 * j;
    float y0, y1, y2;
    rot_t_apply(R, to_f32(q[c]), to_f32(q[c + 1]), to_f32(q[c + 2]), y0, y1, y2);
    qh[c] = from_f32<IO>(y0); qh[c + 1] = from_f32<IO>(y1); qh[c + 2] = from_f32<IO>(y2);
    rot_t_apply(R, to_f32(k[c]), to_f32(k[c + 1]), to_f32(k[c + 2]), y0, y1, y2);
    krow[c] = from_f32<IO>(y0); krow[c + 1] = from_f32<IO>(y1); krow[c + 2] = from_f32<IO>(y2);
    rot_t_apply(R, to_f32(v[c]), to_f32(v[c + 1]), to_f32(v[c + 2]), y0, y1, y2);
    vcol[c * kChunk] = from_f32<IO>(y0);
    vcol[(c + 1) * kChunk] = from_f32<IO>(y1);
    vcol[(c + 2) * kChunk] = from_f32<IO>(y2);
  }
  // dims outside the blocks: leftover dims unrotated, padding zero
  for (int c = 3 * nb + j; c < a.Dp; c += 64) {
    const bool in = c < a.d;
    qh[c] = from_f32<IO>(in ? to_f32(q[c]) : 0.f);
    krow[c] = from_f32<IO>(in ? to_f32(k[c]) : 0.f);
    vcol[c * kChunk] = from_f32<IO>(in ? to_f32(v[c]) : 0.f);
  }
}

// max / sum over the 256 threads of a workgroup (4 waves)
__device__ __forceinline__ float wave_max(float v) {
  static_for<6>([&](auto i) { v = fmaxf(v, __shfl_xor(v, 1 << (int)i)); });
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  static_for<6>([&](auto i) { v += __shfl_xor(v, 1 << (int)i); });
  return v;
}

template <typename T, int DP>
__global__ void __launch_bounds__(256) decode_attn_split(DecodeAttnArgs a) {
  constexpr int E = 16 / sizeof(T);          // elements per 16-byte chunk
  constexpr int CPR = kChunk / E;            // chunks per value-tile row (one dim)
  constexpr int NJ = DP * CPR / 256;         // value-tile chunks per thread
  constexpr int DSTEP = 256 / CPR;           // dims between a thread's chunks
  static_assert(NJ * 256 == DP * CPR, "value tile must split evenly");
  __shared__ float ps[kDecodeSplit];
  __shared__ float red[2][4];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = blockIdx.x % a.nsplit;
  const int64_t bh = blockIdx.x / a.nsplit;
  const int64_t n0 = (int64_t)s * kDecodeSplit;
  const int nk = (int)((a.t + 1 - n0) < kDecodeSplit ? (a.t + 1 - n0) : kDecodeSplit);   // >= 1

  // ---- value tiles of the segment (used after the softmax) ----
  constexpr int kTiles = kDecodeSplit / kChunk;
  u32x4 vraw[kTiles][NJ];
  static_for<kTiles>([&](auto tl) {
    if (tl * kChunk < nk) {
      const u32x4* vt = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.vc) +
                                                       (bh * (a.cap / kChunk) + n0 / kChunk + tl) * DP * kChunk);
      static_for<NJ>([&](auto j) { vraw[tl][j] = vt[tid + 256 * j]; });
    }
  });
  // ---- scores of key n0 + tid (log2 units) ----
  float sc = -INFINITY;
  if (tid < nk) {
    const u32x4* qv = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.qh) + bh * DP);
    const u32x4* kr = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.kc) + (bh * a.cap + n0 + tid) * DP);
    float acc = 0.f;
    static_for<DP / E>([&](auto i) {
      const u32x4 kk = kr[i], qq = qv[i];
      if constexpr (sizeof(T) == 2) {
        static_for<4>([&](auto e) {
          // element copies first: a bit cast of a vector element expression
          // reads the vector's first element whatever the index
          const unsigned ku = kk[(int)e], qu = qq[(int)e];
          acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, ku), __builtin_bit_cast(bf16x2, qu), acc, false);
        });
      } else {
        static_for<4>([&](auto e) { acc = __builtin_fmaf(__uint_as_float(kk[(int)e]), __uint_as_float(qq[(int)e]), acc); });
      }
    });
    sc = acc * a.scale_log2;
  }
  // ---- segment max, weights, segment sum ----
  float m = wave_max(sc);
  if (lane == 0) red[0][w] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float p = tid < nk ? exp2f(sc - m) : 0.f;
  ps[tid] = p;
  float l = wave_sum(p);
  if (lane == 0) red[1][w] = l;
  __syncthreads();
  l = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);

  // ---- P V over the segment's value tiles: chunk c = tid + 256 j of a tile
  // holds dim c / CPR, keys E (c % CPR) .. + E. The chunks do not depend on
  // the scores, so they are loaded with the keys at the start (below, vraw),
  // one memory round trip per workgroup ----
  const int sub = tid % CPR;
  float acc[NJ];
  static_for<NJ>([&](auto j) { acc[j] = 0.f; });
  static_for<kTiles>([&](auto tl) {
    if (tl * kChunk < nk) {
      const int kb = tl * kChunk + E * sub;    // first key of this thread's chunks (segment-local)
      static_for<NJ>([&](auto j) {
        const T* e = reinterpret_cast<const T*>(&vraw[tl][j]);
        static_for<E>([&](auto i) {
          // keys past t hold no data yet: skip them (their weight is zero)
          if (kb + i < nk) acc[j] = __builtin_fmaf(ps[kb + i], to_f32(e[i]), acc[j]);
        });
      });
    }
  });
  static_for<NJ>([&](auto j) {
    for (int o = 1; o < CPR; o <<= 1) acc[j] += __shfl_xor(acc[j], o);
  });
  float* part = a.ws + (bh * a.nsplit + s) * (DP + 2);
  if (tid == 0) { part[0] = m; part[1] = l; }
  if (sub == 0) {
    static_for<NJ>([&](auto j) { part[2 + tid / CPR + DSTEP * j] = acc[j]; });
  }
}

template <typename T, int DP>
__global__ void __launch_bounds__(128) decode_attn_combine(DecodeAttnArgs a) {
  // Merge of the segment partials {m, l, o[DP]}: every load of a 128-segment
  // group is issued before it is used (the weights go through LDS), so the
  // merge costs a few memory round trips, not one per segment.
  constexpr int kTh = 128;
  __shared__ float os[DP];
  __shared__ float wts[kTh];
  __shared__ float red[2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t bh = blockIdx.x;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int ns = (int)a.nsplit;
  const float* part = a.ws + bh * a.nsplit * (DP + 2);
  float M = -INFINITY;
  for (int s = tid; s < ns; s += kTh) M = fmaxf(M, part[(int64_t)s * (DP + 2)]);
  M = wave_max(M);
  if (lane == 0) red[w] = M;
  __syncthreads();
  M = fmaxf(red[0], red[1]);
  float L = 0.f, acc = 0.f;
  for (int base = 0; base < ns; base += kTh) {
    const int n = ns - base < kTh ? ns - base : kTh;
    __syncthreads();                           // the previous group's weights are consumed
    float wgt = 0.f;
    if (tid < n) {
      const float* ps = part + (int64_t)(base + tid) * (DP + 2);
      wgt = exp2f(ps[0] - M);
      L += ps[1] * wgt;
    }
    wts[tid] = wgt;
    __syncthreads();
    if (tid < DP) {
      const float* pc = part + (int64_t)base * (DP + 2) + 2 + tid;
      int s = 0;
      for (; s + 8 <= n; s += 8) {
        float v[8];
        static_for<8>([&](auto i) { v[i] = pc[(int64_t)(s + i) * (DP + 2)]; });
        static_for<8>([&](auto i) { acc = __builtin_fmaf(v[i], wts[s + i], acc); });
      }
      for (; s < n; ++s) acc = __builtin_fmaf(pc[(int64_t)s * (DP + 2)], wts[s], acc);
    }
  }
  L = wave_sum(L);
  __syncthreads();
  if (lane == 0) red[w] = L;
  __syncthreads();
  L = red[0] + red[1];
  if (tid < DP) os[tid] = acc * __builtin_amdgcn_rcpf(L);
  __syncthreads();
  T* orow = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_bs + (int64_t)h * a.o_hs;
  if (tid < a.nb) {
    float y0, y1, y2;
    quat_rotate(load_quat(a.P + (bh * a.nb + tid) * 4), os[3 * tid], os[3 * tid + 1], os[3 * tid + 2], y0, y1, y2);
    orow[3 * tid] = from_f32<T>(y0);
    orow[3 * tid + 1] = from_f32<T>(y1);
    orow[3 * tid + 2] = from_f32<T>(y2);
  }
  for (int c = 3 * a.nb + tid; c < a.d; c += 128) orow[c] = from_f32<T>(os[c]);
}

template <typename IO, typename GT>
hipError_t launch_decode_geom(const DecodeGeomArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((decode_geom<IO, GT>), dim3((unsigned)(a.B * a.H)), dim3(64), 0, s, a);
  return hipGetLastError();
}

template <typename T, int DP>
static hipError_t launch_decode_attn_dp(const DecodeAttnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((decode_attn_split<T, DP>), dim3((unsigned)((int64_t)a.B * a.H * a.nsplit)), dim3(256), 0, s, a);
  hipLaunchKernelGGL((decode_attn_combine<T, DP>), dim3((unsigned)(a.B * a.H)), dim3(128), 0, s, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_decode_attn(const DecodeAttnArgs& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_decode_attn_dp<T, 32>(a, s);
    case 64: return launch_decode_attn_dp<T, 64>(a, s);
    case 96: return launch_decode_attn_dp<T, 96>(a, s);
    default: return hipErrorInvalidValue;
  }
}

int64_t decode_splits(int64_t t) { return (t + kDecodeSplit) / kDecodeSplit; }

template hipError_t launch_decode_geom<float, float>(const DecodeGeomArgs&, hipStream_t);
template hipError_t launch_decode_geom<bf16, float>(const DecodeGeomArgs&, hipStream_t);
template hipError_t launch_decode_geom<bf16, bf16>(const DecodeGeomArgs&, hipStream_t);
template hipError_t launch_decode_attn<float>(const DecodeAttnArgs&, hipStream_t);
template hipError_t launch_decode_attn<bf16>(const DecodeAttnArgs&, hipStream_t);

}  // namespace holo
