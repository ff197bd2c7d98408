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
// Hol^T q^ and a second softmax state, rotated by Hol when the two merge.
//
// Work decomposition as in the causal kernel (4 waves x 32 queries, 64-key
// tiles, S^T = K Q^T and O^T += V^T P^T on 32x32 MFMA tiles). Inert mode is one
// sweep over every key; causal mode sweeps the keys j <= i and then the keys
// j > i, with one query set and one accumulator live at a time (two waves per
// SIMD). The mask arrives as
// bits (one 64-bit word per query row and key tile, packed by pack_mask) and
// as a map of the (128-query, 64-key) tiles it leaves open (mask_tiles): a
// workgroup loads only its open key tiles and a wave skips a tile the mask
// closes for all of its 32 rows, so a sparse mask (the ring mask) costs about
// its diagonal band.
#include <type_traits>

#include "holo_attn_common.h"
#include "holo_dropout.h"

namespace holo {

// one wave per (row, 64-key word): lane l reads allowed(i, 64 w + l) and the
// wave's ballot is the word (keys and rows past T are 0)
__global__ void __launch_bounds__(256) pack_mask(const uint8_t* mask, int64_t rs, int64_t T, int64_t Tp,
                                                 uint64_t* bits) {
  const int64_t nw = Tp / 64;
  const int64_t word = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (word >= Tp * nw) return;                             // uniform over the wave
  const int64_t i = word / nw, key = (word % nw) * 64 + lane;
  const bool on = i < T && key < T && mask[i * rs + key] != 0;
  const uint64_t bal = __ballot(on);
  if (lane == 0) bits[word] = bal;
}

// act[qt][kt] = 1 when the mask allows some pair of query tile qt (128 rows)
// and key tile kt (64 keys): one wave per tile pair, two rows per lane
__global__ void __launch_bounds__(256) mask_tiles(const uint64_t* bits, int64_t T, int64_t Tp, int64_t ntile,
                                                  uint8_t* act) {
  const int64_t nw = Tp / 64;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pair >= ntile * nw) return;                          // uniform over the wave
  const int64_t qt = pair / nw, kt = pair % nw;
  const int64_t r0 = qt * kBM + lane, r1 = r0 + 64;
  uint64_t v = 0;
  if (r0 < T) v |= bits[r0 * nw + kt];
  if (r1 < T) v |= bits[r1 * nw + kt];
  const bool any = __any(v != 0ull);
  if (lane == 0) act[pair] = any;
}

hipError_t launch_pack_mask(const uint8_t* mask, int64_t mask_rs, int64_t T, int64_t Tp, uint64_t* bits,
                            uint8_t* tile_act, hipStream_t s) {
  const int64_t n = Tp * (Tp / 64);
  hipLaunchKernelGGL(pack_mask, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, mask, mask_rs, T, Tp, bits);
  const int64_t ntile = (T + kBM - 1) / kBM, na = ntile * (Tp / 64);
  hipLaunchKernelGGL(mask_tiles, dim3((unsigned)((na + 3) / 4)), dim3(256), 0, s, bits, T, Tp, ntile, tile_act);
  return hipGetLastError();
}

template <typename T, int DP> struct MaskedCfg {
  using C = AttnCfg<T, DP>;
  static constexpr int kStages = 3;
  static constexpr size_t kv_bytes = (size_t)kStages * C::kStage * sizeof(T);
  static constexpr size_t o_bytes = (size_t)kBM * C::OS * sizeof(float);          // staged output
  static constexpr size_t base = ((kv_bytes > o_bytes ? kv_bytes : o_bytes) + 15) / 16 * 16;
  static constexpr int NGR = DP / 3 + 1;                 // 3-dim groups and the leftover dims of a row
  static constexpr int EPI = (kBM * NGR + kThreads - 1) / kThreads;   // epilogue items per thread
  // + the holonomy's quaternions (causal mode) and the workgroup's two lists of
  // open key tiles (base and wrap sweep): a count, then the indices
  static constexpr size_t hol_bytes = (size_t)(DP / 3) * 16;
  static size_t lds(int64_t nkv) { return base + hol_bytes + 8 * (size_t)(nkv + 1); }
};

// One sweep is a pipeline over the workgroup's key tiles j = 0, 1, ... (the
// sweep's key range, less the tiles the mask closes for all of its 128 rows):
// three LDS stages hold tiles j, j+1 and j+2, registers tile j+3 in flight.
// Iteration j computes tile j, stores tile j+2 into the stage tile j-1 used,
// issues the loads of tile j+3 and ends with the tile's barrier. A tile
// holding a wave's diagonal is limited per element to the sweep's side of it
// (the online softmax takes any split of the key set).
//
// Inert mode is one sweep over every key. Causal mode sweeps the base keys
// (j <= i, queries q^) and then the wrap keys (j > i, queries Hol^T q^, rotated
// in registers from q^ between the sweeps); the base sweep's accumulator waits
// in registers and the epilogue merges the two softmax states: with
// m = max(m_b, m_w) the output is
//   P_i (2^(m_b-m) O_b + Hol 2^(m_w-m) O_w) / (2^(m_b-m) l_b + 2^(m_w-m) l_w).
// LSE (the training forward) also writes each row's m + log2 l over both
// branches, for the backward. DROP (with LSE) applies attention dropout: the
// row sums l take every weight, the accumulators only the kept ones, and the
// normalisation multiplies by 1 / (1 - p).
template <typename T, int DP, bool PQ16, bool WRAP, bool LSE = false, bool DROP = false>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 && PQ16 ? 2 : 1)))
attn_masked(typename MaskedArgsOf<LSE>::type a) {
  static_assert(LSE || !DROP, "dropout runs in the training forward");
  using C = AttnCfg<T, DP>;
  using M = MaskedCfg<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  T* const kv = reinterpret_cast<T*>(smem);
  float* const Os = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int lr = lane & 31;
  const int g = lane >> 5;
  // every query tile may visit every key tile; with B*H a multiple of 8 the
  // tiles of one (b, h) run on one XCD (workgroup L runs on XCD L % 8), whose
  // L2 then holds that (b, h)'s keys and values
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

  // ---- the key tiles of each sweep: [lo, hi), less closed tiles ----
  const int nkv_all = (int)(a.Tp / kBN);
  const int64_t q_last = (q0 + kBM < a.T ? q0 + kBM : a.T) - 1;
  const int base_hi = WRAP ? (int)(q_last / kBN) + 1 : nkv_all;
  const int wrap_lo = (int)(q0 / kBN);
  float* const hol_s = reinterpret_cast<float*>(smem + M::base);
  int* const lists = reinterpret_cast<int*>(smem + M::base + M::hol_bytes);
  if (WRAP && tid < a.nb)
    *reinterpret_cast<f32x4*>(hol_s + 4 * tid) = *reinterpret_cast<const f32x4*>(a.hol + ((int64_t)bh * a.nb + tid) * 4);
  if (a.tile_act) {
    if (w < (WRAP ? 2 : 1)) {
      const int lo = w == 0 ? 0 : wrap_lo, hi = w == 0 ? base_hi : nkv_all;
      int* list = lists + w * (nkv_all + 1);
      int cnt = 0;
      for (int base = lo; base < hi; base += 64) {
        const int kt = base + lane;
        const bool on = kt < hi && a.tile_act[(int64_t)qt * nkv_all + kt] != 0;
        const uint64_t bal = __ballot(on);
        if (on) list[1 + cnt + __builtin_popcountll(bal & ((1ull << lane) - 1ull))] = kt;
        cnt += __builtin_popcountll(bal);
      }
      if (lane == 0) list[0] = cnt;
    }
    __syncthreads();
  }

  constexpr bool kBF = sizeof(T) == 2;
  constexpr int QF = kBF ? DP / 16 : DP / 2;
  typedef typename std::conditional<kBF, bf16x8, float>::type qfrag_t;
  const T* const qrow = reinterpret_cast<const T*>(a.qh) + ((int64_t)bh * a.Tp + qi) * DP;
  const bool q_in = qi < a.Tp;                              // rows past Tp read as zero
  qfrag_t qf[QF];
  static_for<QF>([&](auto s) {
    if constexpr (kBF) qf[s] = q_in ? *reinterpret_cast<const bf16x8*>(qrow + 16 * s + 8 * g) : bf16x8{};
    else qf[s] = q_in ? qrow[2 * s + g] : 0.f;
  });
  f32x16 O[DP / 32];
  static_for<DP / 32>([&](auto i) { O[i] = f32x16{}; });
  float m_run = -INFINITY, l_run = 0.f;
  const float c = a.scale_log2;
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
  // scores of the tile in stage st, limited to the mask (mw: this lane's mask
  // word shifted to its element bits), to keys < T and, on a split tile, to
  // the sweep's side of the diagonal (side 0: keys <= query); online softmax;
  // O += V^T P^T
  auto process = [&](int st, int64_t k0, uint64_t mw, bool split, int side) {
    f32x16 S[2];
    {
      const T* Ks = kv + st * C::kStage;
      S[0] = f32x16{}; S[1] = f32x16{};
      static_for<QF>([&](auto s) {
        static_for<2>([&](auto kb) {
          if constexpr (kBF) {
            bf16x8 av = *reinterpret_cast<const bf16x8*>(&Ks[(32 * kb + lr) * C::KS + 16 * s + 8 * g]);
            S[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qf[s], S[kb], 0, 0, 0);
          } else {
            float av = Ks[(32 * kb + lr) * C::KS + 2 * s + g];
            S[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, qf[s], S[kb], 0, 0, 0);
          }
        });
      });
    }
    // element (kb, r) of a lane holds key k0 + 32 kb + 8 (r >> 2) + 4 g + (r & 3)
    const int64_t rel = qi - k0 - 4 * g;                    // off <= rel  <=>  key <= query
    const int64_t lim = a.T - k0 - 4 * g;
    static_for<2>([&](auto kb) {
      static_for<16>([&](auto r) {
        constexpr int off = 32 * kb + 8 * (r >> 2) + (r & 3);
        bool ok = off < lim && ((mw >> off) & 1ull);
        if (split) ok = ok && (side == 0 ? off <= rel : off > rel);
        S[kb][(int)r] = ok ? S[kb][(int)r] * c : -INFINITY;
      });
    });
    const float mx = pair_max(tile_max(S));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;   // nothing allowed yet: every p is 0
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    if (__any(corr != 1.f)) {
      l_run *= corr;
      static_for<DP / 32>([&](auto i) { O[i] *= corr; });
    }
    static_for<2>([&](auto kb) {
      static_for<16>([&](auto r) { S[kb][(int)r] = __builtin_amdgcn_exp2f(S[kb][(int)r] - m_use); });
    });
    const T* Vs = kv + st * C::kStage + kBN * C::KS;
    if constexpr (kBF) {
      // P^T operand in bf16; the row sum is taken over the same rounded values
      bf16x8 pb[2][2];
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          static_for<8>([&](auto e) { pb[kb][hh][(int)e] = (bf16)S[kb][8 * hh + e]; });
        });
      });
      float ls[2][2];
      const bf16x2 one2 = {(bf16)1.f, (bf16)1.f};
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          ls[kb][hh] = 0.f;
          static_for<4>([&](auto e) {
            bf16x2 pr = {pb[kb][hh][2 * e], pb[kb][hh][2 * e + 1]};
            ls[kb][hh] = __builtin_amdgcn_fdot2_f32_bf16(pr, one2, ls[kb][hh], false);
          });
        });
      });
      l_run += (ls[0][0] + ls[0][1]) + (ls[1][0] + ls[1][1]);
      if constexpr (DROP) {
        // elements 4 G .. 4 G + 3 of S[kb]: one query, four consecutive keys
        static_for<2>([&](auto kb) {
          static_for<4>([&](auto G) {
            const u32x4 wd = keep_words(qi, (k0 + 32 * kb + 8 * G + 4 * g) >> 2, bh, a.drop);
            static_for<4>([&](auto e) {
              constexpr int r = 4 * G + e;
              if (wd[(int)e] < a.drop.thr) pb[kb][r >> 3][r & 7] = (bf16)0.f;
            });
          });
        });
      }
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          static_for<DP / 32>([&](auto db) {
            const T* vr = &Vs[(32 * db + lr) * C::VS + 32 * kb + 16 * hh + 4 * g];
            bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
            bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
            bf16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            O[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[kb][hh], O[db], 0, 0, 0);
          });
        });
      });
    } else {
      float t[16];
      static_for<16>([&](auto r) { t[r] = S[0][(int)r] + S[1][(int)r]; });
      static_for<8>([&](auto r) { t[r] += t[r + 8]; });
      static_for<4>([&](auto r) { t[r] += t[r + 4]; });
      static_for<2>([&](auto r) { t[r] += t[r + 2]; });
      l_run += t[0] + t[1];
      if constexpr (DROP) {
        static_for<2>([&](auto kb) {
          static_for<4>([&](auto G) {
            const u32x4 wd = keep_words(qi, (k0 + 32 * kb + 8 * G + 4 * g) >> 2, bh, a.drop);
            static_for<4>([&](auto e) {
              if (wd[(int)e] < a.drop.thr) S[kb][4 * G + e] = 0.f;
            });
          });
        });
      }
      static_for<2>([&](auto kb) {
        static_for<16>([&](auto r) {
          static_for<DP / 32>([&](auto db) {
            float av = Vs[(32 * db + lr) * C::VS + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3)];
            O[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, S[kb][(int)r], O[db], 0, 0, 0);
          });
        });
      });
    }
  };
  // one sweep over key tiles [lo, hi) (or the listed open ones); side 0: keys
  // <= query (the base branch; inert mode: every key), side 1: keys > query
  auto sweep = [&](int side, int lo, int hi, const int* list) __attribute__((always_inline)) {
    const int n = list ? list[0] : hi - lo;
    auto tile_at = [&](int j) { return list ? list[1 + j] : lo + j; };
    // this lane's mask word of a tile (all ones without a mask, 0 past T)
    auto mask_word = [&](int kt) -> uint64_t {
      if (!a.mask_bits) return ~0ull;
      return qi < a.T ? a.mask_bits[qi * nw + kt] : 0ull;
    };
    auto visit = [&](int kt, int st, uint64_t mw) {
      const int64_t k0 = (int64_t)kt * kBN;
      bool need = true, split = false;
      if (WRAP && side == 0) { need = k0 <= qw + 31; split = k0 + kBN - 1 > qw; }
      if (WRAP && side == 1) { need = k0 + kBN - 1 > qw; split = k0 <= qw + 31; }
      if (!need) return;
      // a tile the mask closes for all of the wave's rows changes nothing
      // (every p is 0 and the running max stays): skip it
      if (a.mask_bits && !__any(mw != 0ull)) return;
      process(st, k0, mw >> (4 * g), split, side);
    };
    if (n > 0) { load_tile(tile_at(0)); store_tile(0); }
    if (n > 1) { load_tile(tile_at(1)); store_tile(1); }
    if (n > 2) load_tile(tile_at(2));
    uint64_t mw_next = n > 0 ? mask_word(tile_at(0)) : 0ull;
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const uint64_t mw = mw_next;                          // mask words run one tile ahead
      if (j + 1 < n) mw_next = mask_word(tile_at(j + 1));
      if (wave_live) visit(tile_at(j), j % 3, mw);
      if (j + 2 < n) store_tile((j + 2) % 3);
      if (j + 3 < n) load_tile(tile_at(j + 3));
      __syncthreads();
    }
  };

  sweep(0, 0, base_hi, a.tile_act ? lists : nullptr);
  float sw = 1.f / pair_sum(l_run), sb = 0.f;
  f32x16 Ob[WRAP ? DP / 32 : 1];
  if constexpr (WRAP) {
    // keep the base state, rotate the queries to Hol^T q^ and sweep the wrap keys
    static_for<DP / 32>([&](auto i) { Ob[i] = O[i]; O[i] = f32x16{}; });
    const float m_b = m_run, l_b = pair_sum(l_run);
    m_run = -INFINITY;
    l_run = 0.f;
    {
      float u[DP];
      static_for<DP / C::E>([&](auto cc) {
        const u32x4 raw = q_in ? reinterpret_cast<const u32x4*>(qrow)[cc] : u32x4{0, 0, 0, 0};
        const T* e = reinterpret_cast<const T*>(&raw);
        static_for<C::E>([&](auto j) { u[cc * C::E + j] = to_f32(e[j]); });
      });
      static_for<DP / 3>([&](auto blk) {
        if (blk < a.nb) {
          float y0, y1, y2;
          quat_rotate(qconj(load_quat(hol_s + 4 * blk)), u[3 * blk], u[3 * blk + 1], u[3 * blk + 2], y0, y1, y2);
          u[3 * blk] = to_f32(from_f32<T>(y0));
          u[3 * blk + 1] = to_f32(from_f32<T>(y1));
          u[3 * blk + 2] = to_f32(from_f32<T>(y2));
        }
      });
      static_for<QF>([&](auto s) {
        if constexpr (kBF) {
          static_for<8>([&](auto e) { qf[s][(int)e] = (bf16)(g ? u[16 * s + 8 + e] : u[16 * s + e]); });
        } else {
          qf[s] = g ? u[2 * s + 1] : u[2 * s];
        }
      });
    }
    sweep(1, wrap_lo, nkv_all, a.tile_act ? lists + nkv_all + 1 : nullptr);
    const float l_w = pair_sum(l_run);
    const float m = fmaxf(m_b, m_run);
    const float m_use = m == -INFINITY ? 0.f : m;
    const float ab = __builtin_amdgcn_exp2f(m_b - m_use), aw = __builtin_amdgcn_exp2f(m_run - m_use);
    const float inv = 1.f / (ab * l_b + aw * l_w);
    sb = ab * inv;
    sw = aw * inv;
    if constexpr (LSE) {
      if (g == 0 && qi < a.T) a.lse[(int64_t)bh * a.Tp + qi] = m_use + __log2f(ab * l_b + aw * l_w);
    }
  } else if constexpr (LSE) {
    const float lt = pair_sum(l_run);       // cross-lane: every lane takes part
    if (g == 0 && qi < a.T) a.lse[(int64_t)bh * a.Tp + qi] = m_run + __log2f(lt);
  }
  if constexpr (DROP) {
    sw *= a.drop.scale;
    sb *= a.drop.scale;
  }

  // ---- epilogue: normalise (a row that allowed no key has l = 0: 0 * inf =
  // NaN, as torch.softmax gives), stage, rotate, store. Item = (row, 3-dim
  // group); the rotations of a thread's items are loaded before the LDS work.
  const int ngr = a.nb + (a.d > 3 * a.nb ? 1 : 0);          // 3-dim groups, then the leftover dims
  typedef typename std::conditional<PQ16, u32x2, f32x4>::type pq_t;
  pq_t pq[M::EPI];
  static_for<M::EPI>([&](auto it) {
    const int idx = tid + it * kThreads, r = idx / ngr, gi = idx % ngr;
    const int64_t t = q0 + r;
    if (idx < kBM * ngr && t < a.T && gi < a.nb) {
      if constexpr (PQ16) pq[it] = reinterpret_cast<const u32x2*>(a.P)[(bh * a.T + t) * a.nb + gi];
      else pq[it] = reinterpret_cast<const f32x4*>(a.P)[(bh * a.T + t) * a.nb + gi];
    }
  });
  static_for<DP / 32>([&](auto db) {
    static_for<16>([&](auto r) {
      Os[(32 * w + lr) * C::OS + 32 * db + 8 * (r >> 2) + 4 * g + (r & 3)] = O[db][(int)r] * sw;
    });
  });
  __syncthreads();
  if constexpr (WRAP) {
    // Hol (2^(m_w-m) O_w) in place, then add the base share
    for (int idx = tid; idx < kBM * a.nb; idx += kThreads) {
      const int r = idx / a.nb, gi = idx % a.nb;
      float* u = Os + r * C::OS + 3 * gi;
      float y0, y1, y2;
      quat_rotate(load_quat(hol_s + 4 * gi), u[0], u[1], u[2], y0, y1, y2);
      u[0] = y0; u[1] = y1; u[2] = y2;
    }
    __syncthreads();
    static_for<DP / 32>([&](auto db) {
      static_for<16>([&](auto r) {
        Os[(32 * w + lr) * C::OS + 32 * db + 8 * (r >> 2) + 4 * g + (r & 3)] += Ob[db][(int)r] * sb;
      });
    });
    __syncthreads();
  }
  static_for<M::EPI>([&](auto it) {
    const int idx = tid + it * kThreads, r = idx / ngr, gi = idx % ngr;
    const int64_t t = q0 + r;
    if (idx >= kBM * ngr || t >= a.T) return;
    T* orow = reinterpret_cast<T*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs;
    const float* u = Os + r * C::OS;
    if (gi < a.nb) {
      quat q;
      if constexpr (PQ16) q = unpack_quat_snorm16(pq[it]);
      else q = quat{pq[it][0], pq[it][1], pq[it][2], pq[it][3]};
      if (!WRAP) q = qconj(q);                               // inert: P_i^T
      float y0, y1, y2;
      quat_rotate(q, u[3 * gi], u[3 * gi + 1], u[3 * gi + 2], y0, y1, y2);
      orow[3 * gi] = from_f32<T>(y0);
      orow[3 * gi + 1] = from_f32<T>(y1);
      orow[3 * gi + 2] = from_f32<T>(y2);
    } else {
      for (int cc = 3 * a.nb; cc < a.d; ++cc) orow[cc] = from_f32<T>(u[cc]);
    }
  });
}

template <typename T, int DP, bool PQ16, bool WRAP, bool LSE = false, bool DROP = false>
static hipError_t launch_masked_dp(const typename MaskedArgsOf<LSE>::type& a, hipStream_t s) {
  using M = MaskedCfg<T, DP>;
  const size_t lds = M::lds(a.Tp / kBN);
  if (lds > (size_t)kMaxDynamicLds) return hipErrorInvalidValue;
  const hipError_t attr = allow_dynamic_lds<&attn_masked<T, DP, PQ16, WRAP, LSE, DROP>>();
  if (attr != hipSuccess) return attr;
  const int64_t ntile = (a.T + kBM - 1) / kBM;
  hipLaunchKernelGGL((attn_masked<T, DP, PQ16, WRAP, LSE, DROP>), dim3((unsigned)(a.B * a.H * ntile)),
                     dim3(kThreads), lds, s, a);
  return hipGetLastError();
}

template <typename T, bool PQ16, bool WRAP, bool LSE = false, bool DROP = false>
static hipError_t launch_masked_pf(const typename MaskedArgsOf<LSE>::type& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_masked_dp<T, 32, PQ16, WRAP, LSE, DROP>(a, s);
    case 64: return launch_masked_dp<T, 64, PQ16, WRAP, LSE, DROP>(a, s);
    case 96: return launch_masked_dp<T, 96, PQ16, WRAP, LSE, DROP>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t launch_attn_masked(const MaskedArgs& a, hipStream_t s) {
  const bool wrap = a.mode == 0;
  if (a.p_format) return wrap ? launch_masked_pf<T, true, true>(a, s) : launch_masked_pf<T, true, false>(a, s);
  return wrap ? launch_masked_pf<T, false, true>(a, s) : launch_masked_pf<T, false, false>(a, s);
}

// the training forward: fp32 quaternions (the backward's format) and the LSE;
// with dropout, its own instantiations
template <typename T>
hipError_t launch_attn_masked_lse(const MaskedLseArgs& a, hipStream_t s) {
  if (a.p_format) return hipErrorInvalidValue;
  if (a.dropout)
    return a.mode == 0 ? launch_masked_pf<T, false, true, true, true>(a, s)
                       : launch_masked_pf<T, false, false, true, true>(a, s);
  return a.mode == 0 ? launch_masked_pf<T, false, true, true>(a, s) : launch_masked_pf<T, false, false, true>(a, s);
}

template hipError_t launch_attn_masked<float>(const MaskedArgs&, hipStream_t);
template hipError_t launch_attn_masked<bf16>(const MaskedArgs&, hipStream_t);
template hipError_t launch_attn_masked_lse<float>(const MaskedLseArgs&, hipStream_t);
template hipError_t launch_attn_masked_lse<bf16>(const MaskedLseArgs&, hipStream_t);

}  // namespace holo
