// Path-ordered attention for any mask and either mode on gfx950 MFMA: the
// reference's exact path (kernel/attention_fast.py:129-166, equal to the
// definition core/attention.py:156-192), which the reference's kernel module
// runs for every call off its causal + tril kernel path
// (kernel/attention_kernel.py:203-213).
//
// The reference transports key/value j to query i by
//   causal: G_arc[i, j] = P_i P_j^T (i >= j),  P_i Hol P_j^T (i < j)
//   inert:  G_arc[i, j] = P_i^T P_j
// masks disallowed scores with -inf and takes torch.softmax (a row that
// allows no key is NaN). In transported coordinates, with the scan writing
// u^ = P^T u (causal) or u' = P u (inert):
//   causal: s_ij = q^_i . k^_j (i >= j),  (Hol^T q^_i) . k^_j (i < j)
//           o_i  = P_i (sum_{j<=i} a_ij v^_j + Hol sum_{j>i} a_ij v^_j)
//   inert:  s_ij = q'_i . k'_j,   o_i = P_i^T sum_j a_ij v'_j
// so the wrap branch needs no second key/value copy: a second query set
// Hol^T q^ (written once per call by wrap_queries) and a second accumulator,
// rotated by Hol in the epilogue.
//
// Work decomposition as in the causal kernel (4 waves x 32 queries, 64-key
// tiles, S^T = K Q^T and O^T += V^T P^T on 32x32 MFMA tiles), over every key
// tile. Per tile and wave the base scores are computed when some key of the
// tile is <= some query of the wave, the wrap scores when some key is later
// (causal mode), and diagonal tiles select per element. The mask arrives as
// bits (one 64-bit word per query row and key tile, packed by pack_mask).
#include <type_traits>

#include "holo_attn_common.h"

namespace holo {

__global__ void __launch_bounds__(256) pack_mask(const uint8_t* mask, int64_t rs, int64_t T, int64_t Tp,
                                                 uint64_t* bits) {
  const int64_t nw = Tp / 64;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= Tp * nw) return;
  const int64_t i = gid / nw, w = gid % nw;
  uint64_t v = 0;
  if (i < T) {
    const uint8_t* row = mask + i * rs + 64 * w;
    const int n = T - 64 * w < 64 ? (int)(T - 64 * w) : 64;
    for (int e = 0; e < n; ++e) v |= (uint64_t)(row[e] != 0) << e;
  }
  bits[gid] = v;
}

hipError_t launch_pack_mask(const uint8_t* mask, int64_t mask_rs, int64_t T, int64_t Tp, uint64_t* bits,
                            hipStream_t s) {
  const int64_t n = Tp * (Tp / 64);
  hipLaunchKernelGGL(pack_mask, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, mask, mask_rs, T, Tp, bits);
  return hipGetLastError();
}

// qhw = Hol^T qh on every 3-dim block of every row (B, H, Tp, Dp); the
// remaining dims (d - 3 nb and the padding) are copied.
template <typename T>
__global__ void __launch_bounds__(256) wrap_queries(MaskedArgs a, T* qhw) {
  const int ng = (a.Dp + 2) / 3;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)a.B * a.H * a.Tp;
  if (gid >= rows * ng) return;
  const int64_t row = gid / ng;
  const int gi = (int)(gid % ng);
  const int64_t bh = row / a.Tp;
  const T* src = reinterpret_cast<const T*>(a.qh) + row * a.Dp + 3 * gi;
  T* dst = qhw + row * a.Dp + 3 * gi;
  if (gi < a.nb) {
    float y0, y1, y2;
    quat_rotate(qconj(load_quat(a.hol + (bh * a.nb + gi) * 4)), to_f32(src[0]), to_f32(src[1]), to_f32(src[2]),
                y0, y1, y2);
    dst[0] = from_f32<T>(y0); dst[1] = from_f32<T>(y1); dst[2] = from_f32<T>(y2);
  } else {
    for (int c = 0; c < 3 && 3 * gi + c < a.Dp; ++c) dst[c] = src[c];
  }
}

template <typename T>
hipError_t launch_wrap_queries(const MaskedArgs& a, void* qhw, hipStream_t s) {
  const int64_t n = (int64_t)a.B * a.H * a.Tp * ((a.Dp + 2) / 3);
  hipLaunchKernelGGL(wrap_queries<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a,
                     reinterpret_cast<T*>(qhw));
  return hipGetLastError();
}

template <typename T, int DP> struct MaskedCfg {
  using C = AttnCfg<T, DP>;
  static constexpr int kStages = 2;
  static constexpr size_t kv_bytes = (size_t)kStages * C::kStage * sizeof(T);
  static constexpr size_t o_bytes = (size_t)2 * kBM * C::OS * sizeof(float);   // base and wrap outputs
  static constexpr size_t lds = kv_bytes > o_bytes ? kv_bytes : o_bytes;
};

// Two-stage pipeline over all key tiles: iteration j loads tile j+1 into
// registers, computes tile j from LDS stage j%2, stores tile j+1 into the
// other stage and ends with the tile's barrier.
template <typename T, int DP, bool PQ16, bool WRAP>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1)))
attn_masked(MaskedArgs a) {
  using C = AttnCfg<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  T* const kv = reinterpret_cast<T*>(smem);
  float* const Obs = reinterpret_cast<float*>(smem);
  float* const Ows = Obs + kBM * C::OS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int lr = lane & 31;
  const int g = lane >> 5;
  // every query tile visits every key tile; with B*H a multiple of 8 the tiles
  // of one (b, h) run on one XCD (workgroup L runs on XCD L % 8), whose L2
  // then holds that (b, h)'s keys and values
  const int ntile = (int)((a.T + kBM - 1) / kBM);
  const int L = blockIdx.x;
  int bh, qt;
  if ((a.B * a.H) % 8 == 0) {
    const int j = L >> 3;
    bh = 8 * (j / ntile) + (L & 7);
    qt = j % ntile;
  } else {
    bh = L / ntile;
    qt = L % ntile;
  }
  const int b = bh / a.H, h = bh % a.H;
  const int64_t q0 = (int64_t)qt * kBM;
  const int64_t qw = q0 + 32 * w;
  const int64_t qi = qw + lr;                               // this lane's query

  constexpr bool kBF = sizeof(T) == 2;
  constexpr int QF = kBF ? DP / 16 : DP / 2;
  typedef typename std::conditional<kBF, bf16x8, float>::type qfrag_t;
  qfrag_t qf[QF], qwf[WRAP ? QF : 1];
  {
    const bool in = qi < a.Tp;                              // rows past Tp read as zero
    const T* qrow = reinterpret_cast<const T*>(a.qh) + ((int64_t)bh * a.Tp + qi) * DP;
    const T* wrow = reinterpret_cast<const T*>(a.qhw) + ((int64_t)bh * a.Tp + qi) * DP;
    static_for<QF>([&](auto s) {
      if constexpr (kBF) {
        qf[s] = in ? *reinterpret_cast<const bf16x8*>(qrow + 16 * s + 8 * g) : bf16x8{};
        if constexpr (WRAP) qwf[s] = in ? *reinterpret_cast<const bf16x8*>(wrow + 16 * s + 8 * g) : bf16x8{};
      } else {
        qf[s] = in ? qrow[2 * s + g] : 0.f;
        if constexpr (WRAP) qwf[s] = in ? wrow[2 * s + g] : 0.f;
      }
    });
  }
  f32x16 Ob[DP / 32], Ow[WRAP ? DP / 32 : 1];
  static_for<DP / 32>([&](auto i) { Ob[i] = f32x16{}; });
  static_for<(WRAP ? DP / 32 : 1)>([&](auto i) { Ow[i] = f32x16{}; });
  float m_run = -INFINITY, l_run = 0.f;
  const float c = a.scale_log2;
  const int nkv = (int)(a.Tp / kBN);
  const int64_t nw = a.Tp / 64;                             // mask words per row
  const bool wave_live = qw < a.T;

  const u32x4* kbase = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.kh) + (int64_t)bh * a.Tp * DP);
  const u32x4* vbase = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.vh_t) + (int64_t)bh * a.Tp * DP);
  constexpr int TCH = kBN * DP / C::E;
  constexpr int RC = DP / C::E, VC = kBN / C::E;
  u32x4 kreg[C::KCH], vreg[C::VCH];
  auto load_tile = [&](int kt) {
    static_for<C::KCH>([&](auto j) { kreg[j] = kbase[(int64_t)kt * TCH + tid + j * kThreads]; });
    static_for<C::VCH>([&](auto j) { vreg[j] = vbase[(int64_t)kt * TCH + tid + j * kThreads]; });
  };
  auto store_tile = [&](int st) {
    T* Ks = kv + st * C::kStage;
    T* Vs = Ks + kBN * C::KS;
    static_for<C::KCH>([&](auto j) {
      const int i = tid + j * kThreads, r = i / RC, cc = i % RC;
      *reinterpret_cast<u32x4*>(&Ks[r * C::KS + cc * C::E]) = kreg[j];
    });
    static_for<C::VCH>([&](auto j) {
      const int i = tid + j * kThreads, r = i / VC, cc = i % VC;
      u32x2* dst = reinterpret_cast<u32x2*>(&Vs[r * C::VS + cc * C::E]);
      dst[0] = vreg[j].xy;
      dst[1] = vreg[j].zw;
    });
  };
  auto qk = [&](int st, const qfrag_t (&q)[QF], f32x16 (&S)[2]) {
    const T* Ks = kv + st * C::kStage;
    S[0] = f32x16{}; S[1] = f32x16{};
    static_for<QF>([&](auto s) {
      static_for<2>([&](auto kb) {
        if constexpr (kBF) {
          bf16x8 av = *reinterpret_cast<const bf16x8*>(&Ks[(32 * kb + lr) * C::KS + 16 * s + 8 * g]);
          S[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, q[s], S[kb], 0, 0, 0);
        } else {
          float av = Ks[(32 * kb + lr) * C::KS + 2 * s + g];
          S[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, q[s], S[kb], 0, 0, 0);
        }
      });
    });
  };
  // O^T += V^T P^T for one accumulator set; P given per element in fp32
  auto pv = [&](int st, const float (&p)[32], f32x16 (&O)[DP / 32]) {
    const T* Vs = kv + st * C::kStage + kBN * C::KS;
    if constexpr (kBF) {
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          bf16x8 pb;
          static_for<8>([&](auto e) { pb[(int)e] = (bf16)p[16 * kb + 8 * hh + e]; });
          static_for<DP / 32>([&](auto db) {
            const T* vr = &Vs[(32 * db + lr) * C::VS + 32 * kb + 16 * hh + 4 * g];
            bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
            bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
            bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            O[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb, O[db], 0, 0, 0);
          });
        });
      });
    } else {
      static_for<2>([&](auto kb) {
        static_for<16>([&](auto r) {
          static_for<DP / 32>([&](auto db) {
            float av = Vs[(32 * db + lr) * C::VS + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3)];
            O[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, p[16 * kb + r], O[db], 0, 0, 0);
          });
        });
      });
    }
  };
  auto process = [&](int kt, int st) {
    const int64_t k0 = (int64_t)kt * kBN;
    // element (kb, r) of a lane holds key k0 + 32 kb + 8 (r >> 2) + 4 g + (r & 3)
    const int64_t rel = qi - k0 - 4 * g;                  // key offset limit of the base branch
    const int64_t lim = a.T - k0 - 4 * g;                 // keys past T do not exist
    const bool any_base = !WRAP || k0 <= qw + 31;         // some key <= some query of the wave
    const bool any_wrap = WRAP && k0 + kBN - 1 > qw;      // some key > some query of the wave
    f32x16 Sb[2], Sw[2];
    if (any_base) qk(st, qf, Sb);
    else { Sb[0] = f32x16{}; Sb[1] = f32x16{}; }
    if constexpr (WRAP) {
      if (any_wrap) qk(st, qwf, Sw);
      else { Sw[0] = f32x16{}; Sw[1] = f32x16{}; }
    }
    uint64_t mw = ~0ull;
    if (a.mask_bits) mw = qi < a.T ? a.mask_bits[qi * nw + kt] : 0ull;
    mw >>= 4 * g;
    float s[32];
    bool base[32];
    static_for<2>([&](auto kb) {
      static_for<16>([&](auto r) {
        constexpr int off = 32 * kb + 8 * (r >> 2) + (r & 3);
        constexpr int bit = 32 * kb + 8 * (r >> 2) + (r & 3);
        const bool is_base = !WRAP || off <= rel;
        float v = Sb[kb][(int)r];
        if constexpr (WRAP) v = is_base ? v : Sw[kb][(int)r];
        const bool ok = off < lim && ((mw >> bit) & 1ull);
        s[16 * kb + r] = ok ? v * c : -INFINITY;
        base[16 * kb + r] = is_base;
      });
    });
    float mx = s[0];
    static_for<31>([&](auto i) { mx = fmaxf(mx, s[i + 1]); });
    mx = pair_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;   // no key allowed yet: every p is 0
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    l_run *= corr;
    static_for<DP / 32>([&](auto i) { Ob[i] *= corr; });
    if constexpr (WRAP) static_for<DP / 32>([&](auto i) { Ow[i] *= corr; });
    float pb[32], pw[32];
    float ls = 0.f;
    static_for<32>([&](auto i) {
      float p = __builtin_amdgcn_exp2f(s[i] - m_use);
      if constexpr (kBF) p = (float)(bf16)p;          // the row sum uses the values the MFMA consumes
      ls += p;
      pb[i] = base[i] ? p : 0.f;
      pw[i] = base[i] ? 0.f : p;
    });
    l_run += ls;
    if (any_base) pv(st, pb, Ob);
    if constexpr (WRAP) {
      if (any_wrap) pv(st, pw, Ow);
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int j = 0; j < nkv; ++j) {
    if (j + 1 < nkv) load_tile(j + 1);
    if (wave_live) process(j, j & 1);
    if (j + 1 < nkv) store_tile((j + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: normalise (a row that allowed no key has l = 0: 0 * inf =
  // NaN, as torch.softmax gives), stage both accumulators, combine, rotate ----
  const float inv = 1.f / pair_sum(l_run);
  static_for<DP / 32>([&](auto db) {
    static_for<16>([&](auto r) {
      const int idx = (32 * w + lr) * C::OS + 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
      Obs[idx] = Ob[db][(int)r] * inv;
      if constexpr (WRAP) Ows[idx] = Ow[db][(int)r] * inv;
    });
  });
  __syncthreads();
  const int ngr = a.nb + (a.d > 3 * a.nb ? 1 : 0);          // 3-dim groups, then the leftover dims
  for (int idx = tid; idx < kBM * ngr; idx += kThreads) {
    const int r = idx / ngr, gi = idx % ngr;
    const int64_t t = q0 + r;
    if (t >= a.T) continue;
    T* orow = reinterpret_cast<T*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs;
    const float* ob = Obs + r * C::OS;
    const float* ow = Ows + r * C::OS;
    if (gi < a.nb) {
      float u0 = ob[3 * gi], u1 = ob[3 * gi + 1], u2 = ob[3 * gi + 2];
      if constexpr (WRAP) {
        float w0, w1, w2;
        quat_rotate(load_quat(a.hol + ((int64_t)bh * a.nb + gi) * 4), ow[3 * gi], ow[3 * gi + 1], ow[3 * gi + 2],
                    w0, w1, w2);
        u0 += w0; u1 += w1; u2 += w2;
      }
      quat pq;
      if constexpr (PQ16) {
        pq = unpack_quat_snorm16(reinterpret_cast<const u32x2*>(a.P)[(bh * a.T + t) * a.nb + gi]);
      } else {
        pq = load_quat(reinterpret_cast<const float*>(a.P) + ((bh * a.T + t) * a.nb + gi) * 4);
      }
      if (a.mode != 0) pq = qconj(pq);                       // inert: P_i^T
      float y0, y1, y2;
      quat_rotate(pq, u0, u1, u2, y0, y1, y2);
      orow[3 * gi] = from_f32<T>(y0);
      orow[3 * gi + 1] = from_f32<T>(y1);
      orow[3 * gi + 2] = from_f32<T>(y2);
    } else {
      for (int cc = 3 * a.nb; cc < a.d; ++cc) orow[cc] = from_f32<T>(WRAP ? ob[cc] + ow[cc] : ob[cc]);
    }
  }
}

template <typename T, int DP, bool PQ16, bool WRAP>
static hipError_t launch_masked_dp(const MaskedArgs& a, hipStream_t s) {
  using M = MaskedCfg<T, DP>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&attn_masked<T, DP, PQ16, WRAP>), hipFuncAttributeMaxDynamicSharedMemorySize,
      (int)M::lds);
  if (attr != hipSuccess) return attr;
  const int64_t ntile = (a.T + kBM - 1) / kBM;
  hipLaunchKernelGGL((attn_masked<T, DP, PQ16, WRAP>), dim3((unsigned)(a.B * a.H * ntile)), dim3(kThreads),
                     M::lds, s, a);
  return hipGetLastError();
}

template <typename T, bool PQ16, bool WRAP>
static hipError_t launch_masked_pf(const MaskedArgs& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_masked_dp<T, 32, PQ16, WRAP>(a, s);
    case 64: return launch_masked_dp<T, 64, PQ16, WRAP>(a, s);
    case 96: return launch_masked_dp<T, 96, PQ16, WRAP>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t launch_attn_masked(const MaskedArgs& a, hipStream_t s) {
  const bool wrap = a.mode == 0;
  if (a.p_format) return wrap ? launch_masked_pf<T, true, true>(a, s) : launch_masked_pf<T, true, false>(a, s);
  return wrap ? launch_masked_pf<T, false, true>(a, s) : launch_masked_pf<T, false, false>(a, s);
}

template hipError_t launch_wrap_queries<float>(const MaskedArgs&, void*, hipStream_t);
template hipError_t launch_wrap_queries<bf16>(const MaskedArgs&, void*, hipStream_t);
template hipError_t launch_attn_masked<float>(const MaskedArgs&, hipStream_t);
template hipError_t launch_attn_masked<bf16>(const MaskedArgs&, hipStream_t);

}  // namespace holo
