// Backward of the exact path (any mask; causal mode with the wrap branch
// through the holonomy, or inert mode) on gfx950: the gradient that torch
// autograd takes through the reference's exact path (kernel/attention_fast.py:
// 78-166, which kernel/attention_kernel.py:211-213 runs off its kernel path).
//
// Causal mode, in the path frame (u^ = P^T u), pairs i >= j (base) and i < j
// (wrap, through Hol): with qw = Hol^T q^ and dow = Hol^T do^,
//   s_ij = scale q^_i . k^_j (base), scale qw_i . k^_j (wrap)
//   dS = Pm (dP - delta), dP_ij = do^_i . v^_j (base), dow_i . v^_j (wrap)
//   dq^ = scale (dS_base k^ + Hol dS_wrap k^)      (the wrap term as dqw)
//   dk^ = scale (dS_base^T q^ + dS_wrap^T qw),   dv^ = Pm_base^T do^ + Pm_wrap^T dow.
// The per-token cross sums of link_bwd stand as in the tril path (with the
// full outputs and gradients); Hol = G_{T-1} P_{T-1} is P_T of the link
// recursion, so its cross sum c_hol = sum_j k^_j x dkw_j + v^_j x dvw_j (the
// wrap branch's dK^, dV^) seeds the suffix at the last chunk and gives the
// closing edge its gradient. Inert mode (u' = P u) is the same algebra with
// P replaced by P^T: one branch over every allowed pair, c = -P^T c', the
// gradients returned by P^T, no holonomy.
//
// Kernels, in launch order: bwd_prep (doh or doh', delta, vh rows; causal:
// qw, dow), attn_bwd_masked_dkdv (per 128 keys: the wrap sweep over queries
// before the keys, its dK, dV stored apart, then the base sweep on top),
// attn_bwd_masked_dq (per 128 queries: base sweep, then the wrap sweep with
// qw, dow stored as dqw), hol_torque (causal), link_bwd.
#include "holo_bwd_kernels.h"
#include "holo_dropout.h"

namespace holo {

// ---------------------------------------------------------------------------
// exact path: attention backward for any mask, causal mode (the wrap branch
// through the holonomy) or inert mode
// ---------------------------------------------------------------------------
// A sweep covers one branch's pairs, each further limited to the mask:
//   kRelBase  i >= j (causal base branch), operands q^, do^
//   kRelWrap  i <  j (causal wrap branch), operands qw = Hol^T q^, dow = Hol^T do^
//   kRelAll   every pair (inert mode), operands q', do'
// With the forward's LSE over both branches the probabilities and dS of each
// pair follow as in the causal kernels; the wrap branch's dK and dV (in the
// frame of k^ and v^) are the sums over its pairs, so one accumulator carries
// both branches. The wrap branch's share of dK, dV (for the holonomy's
// torque) and its dQ (in the frame of qw, rotated back by Hol in link_bwd)
// are also stored apart. DROP: the forward's attention dropout (z = keep /
// (1 - p) per pair, regenerated from its seed): dV takes p z, and
// dS = p (z dP - delta) (delta = do . o already holds the dropped output).
enum : int { kRelBase = 0, kRelWrap = 1, kRelAll = 2 };
constexpr int kMapRows = 128;        // query rows per tile of the open-tile map (mask_tiles)

template <typename T, int DP, bool WRAP, bool DROP = false>
__global__ void __launch_bounds__(kBwdThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 2 : 1)))
attn_bwd_masked_dkdv(MaskedBwdArgs a) {
  using C = BwdCfg<T, DP, kFillKV>;
  typedef typename frag<T>::type frag_t;
  constexpr bool kBF = sizeof(T) == 2;
  using M = typename TileCopy<T, DP, kFillKV>::template Multi<2, kBF ? 0 : 2>;
  __shared__ __align__(16) T tiles[M::kElems];
  __shared__ float lse_s[kFillKV], del_s[kFillKV];
  __shared__ uint64_t mw_s[kFillKV][2];            // the fill rows' mask words over the workgroup's 128 keys
  __shared__ __align__(16) T Kw[128 * C::RS];
  const T* const Qs = tiles;
  const T* const dOs = tiles + M::kRowTile;
  const T* const QTs = tiles + 2 * M::kRowTile;
  const T* const dOTs = tiles + 2 * M::kRowTile + M::kColTile;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t kb = blockIdx.x / nbh, bh = blockIdx.x % nbh;
  const int64_t k0 = kb * 128, kw0 = k0 + 32 * w;
  const bool wave_in = kw0 < a.T;
  const int64_t nw = a.Tp / 64;                    // mask words per row

  frag_t vf[C::QF];
  {
    const bool in = kw0 < a.Tp;
    const T* vrow = reinterpret_cast<const T*>(a.vh) + (bh * a.Tp + kw0 + lr) * DP;
    static_for<C::QF>([&](auto s) {
      if constexpr (kBF) vf[s] = in ? *reinterpret_cast<const bf16x8*>(vrow + 16 * s + 8 * g) : bf16x8{};
      else vf[s] = in ? vrow[2 * s + g] : 0.f;
    });
    constexpr int E = C::E, RCH = DP / E;
    for (int i = tid; i < 128 * RCH; i += kBwdThreads) {
      const int r = i / RCH, cc = i % RCH;
      const bool rin = k0 + r < a.Tp;
      const u32x4 v = rin ? *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.kh) + (bh * a.Tp + k0 + r) * DP + cc * E)
                          : u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&Kw[r * C::RS + cc * E]) = v;
    }
  }
  f32x16 dK[DP / 32], dV[DP / 32];
  static_for<DP / 32>([&](auto i) { dK[i] = f32x16{}; dV[i] = f32x16{}; });
  const float cl = a.scale_log2;
  const int64_t key = kw0 + lr;
  const int kword = w >> 1, kbit = 32 * (w & 1) + lr;   // this lane's key in the workgroup's two mask words

  // one branch over the query fills covering [qlo, qhi)
  auto sweep = [&](const void* qsrc, const void* dsrc, const void* qtsrc, const void* dtsrc, int64_t qlo,
                   int64_t qhi, auto rel_c) {
    constexpr int rel = decltype(rel_c)::value;
    if (qhi <= qlo) return;
    const int f0 = (int)(qlo / kFillKV), f1 = (int)((qhi + kFillKV - 1) / kFillKV);
    u32x4 r[M::IT];
    float ls = INFINITY, dl = 0.f;
    uint64_t mwr = 0ull;
    auto load_fill = [&](int qf) {
      const int64_t q0 = (int64_t)qf * kFillKV;
      const int64_t tile = (bh * a.nch + q0 / kChunk) * DP * kChunk;
      const T* const rows[2] = {reinterpret_cast<const T*>(qsrc) + (bh * a.Tp + q0) * DP,
                                reinterpret_cast<const T*>(dsrc) + (bh * a.Tp + q0) * DP};
      const T* const cols[2] = {kBF ? nullptr : reinterpret_cast<const T*>(qtsrc) + tile,
                                kBF ? nullptr : reinterpret_cast<const T*>(dtsrc) + tile};
      M::load(r, rows, cols, (int)(q0 % kChunk), tid);
      const bool qin = tid < kFillKV && q0 + tid < a.T;
      ls = qin ? a.lse[bh * a.Tp + q0 + tid] : INFINITY;
      dl = qin ? a.delta[bh * a.Tp + q0 + tid] : 0.f;
      if (tid < 2 * kFillKV) {
        const int64_t qrow = q0 + (tid >> 1), wd = k0 / 64 + (tid & 1);
        mwr = a.mask_bits == nullptr ? ~0ull : (qrow < a.T && wd < nw ? a.mask_bits[qrow * nw + wd] : 0ull);
      }
    };
    auto store_fill = [&]() {
      M::store(tiles, r, tid);
      if (tid < kFillKV) { lse_s[tid] = ls; del_s[tid] = dl; }
      if (tid < 2 * kFillKV) mw_s[tid >> 1][tid & 1] = mwr;
    };
    // the first fill at or after qf that the mask opens for the workgroup's
    // keys (the map of open (128-query, 64-key) tiles; every thread reads the
    // same bytes, so the walk is uniform)
    auto open_from = [&](int qf) {
      if (a.tile_act == nullptr) return qf;
      const int64_t kt0 = k0 / 64;
      for (; qf < f1; ++qf) {
        const int64_t row = (int64_t)qf * kFillKV / kMapRows * nw;
        if (a.tile_act[row + kt0] != 0 || (kt0 + 1 < nw && a.tile_act[row + kt0 + 1] != 0)) break;
      }
      return qf;
    };
    const int first = open_from(f0);
    if (first >= f1) return;                // uniform: no open pair in this sweep
    __syncthreads();                        // the previous sweep is done with the tiles
    load_fill(first);
    store_fill();
    __syncthreads();
    for (int qf = first; qf < f1;) {
      const int64_t q0 = (int64_t)qf * kFillKV;
      const int nxt = open_from(qf + 1);
      if (nxt < f1) load_fill(nxt);
      static_for<kFillKV / kBT>([&](auto sub) {
        const int64_t qs0 = q0 + kBT * sub;
        if (!wave_in) return;
        if (rel == kRelBase && qs0 + kBT - 1 < kw0) return;    // every query before every key of the wave
        if (rel == kRelWrap && qs0 >= kw0 + kBT - 1) return;   // no query before any key of the wave
        const int ro = kBT * sub;
        if (a.mask_bits != nullptr) {
          // a sub-tile the mask closes for every pair of the wave adds only
          // zeros: skip it (uniform over the wave)
          bool open = false;
          static_for<16>([&](auto rr) {
            const int qr = 8 * (rr >> 2) + 4 * g + (rr & 3);
            open = open || ((mw_s[ro + qr][kword] >> kbit) & 1ull) != 0ull;
          });
          if (!__any(open)) return;
        }
        f32x16 S = f32x16{}, dP = f32x16{};
        static_for<C::QF>([&](auto s) {
          if constexpr (kBF) {
            const bf16x8 qa = *reinterpret_cast<const bf16x8*>(&Qs[(ro + lr) * C::RS + 16 * s + 8 * g]);
            const bf16x8 da = *reinterpret_cast<const bf16x8*>(&dOs[(ro + lr) * C::RS + 16 * s + 8 * g]);
            const bf16x8 kbv = *reinterpret_cast<const bf16x8*>(&Kw[(32 * w + lr) * C::RS + 16 * s + 8 * g]);
            S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kbv, S, 0, 0, 0);
            dP = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vf[s], dP, 0, 0, 0);
          } else {
            S = __builtin_amdgcn_mfma_f32_32x32x2f32(Qs[(ro + lr) * C::RS + 2 * s + g], Kw[(32 * w + lr) * C::RS + 2 * s + g], S, 0, 0, 0);
            dP = __builtin_amdgcn_mfma_f32_32x32x2f32(dOs[(ro + lr) * C::RS + 2 * s + g], vf[s], dP, 0, 0, 0);
          }
        });
        // dropout: this lane's words for its key at the 16 queries. Philox
        // call (query, key / 4) gives the words of four consecutive keys, held
        // by the lanes of one quad; in group G each lane c = lane % 4 of a
        // quad draws for query qs0 + 8 G + 4 g + c, and four rotations
        // (step s: lane c sends word (c - s) % 4, receives from lane
        // (c + s) % 4) give every lane its own key's word of each query.
        float z[DROP ? 16 : 1];
        if constexpr (DROP) {
          const int c = lr & 3;
          static_for<4>([&](auto G) {
            const u32x4 wd = keep_words(qs0 + 8 * G + 4 * g + c, key >> 2, bh, a.drop);
            u32x4 got;
            static_for<4>([&](auto st) {
              got[(int)st] = __shfl((int)pick4(wd, (c - (int)st) & 3), (lane & ~3) | ((c + (int)st) & 3));
            });
            static_for<4>([&](auto e) {          // query qs0 + 8 G + 4 g + e arrived at step (e - c) % 4
              z[4 * G + e] = pick4(got, ((int)e - c) & 3) >= a.drop.thr ? a.drop.scale : 0.f;
            });
          });
        }
        // element r: query qs0 + qr (row), this lane's key (column)
        static_for<16>([&](auto rr) {
          const int qr = 8 * (rr >> 2) + 4 * g + (rr & 3);
          const int64_t qi = qs0 + qr;
          bool ok = key < a.T && ((mw_s[ro + qr][kword] >> kbit) & 1ull) != 0ull;
          if constexpr (rel == kRelBase) ok = ok && key <= qi;
          if constexpr (rel == kRelWrap) ok = ok && key > qi;
          const float pm = ok ? exp2f(__builtin_fmaf(S[(int)rr], cl, -lse_s[ro + qr])) : 0.f;
          if constexpr (DROP) {
            S[(int)rr] = pm * z[(int)rr];
            dP[(int)rr] = ok ? pm * (z[(int)rr] * dP[(int)rr] - del_s[ro + qr]) : 0.f;
          } else {
            S[(int)rr] = pm;
            dP[(int)rr] = ok ? pm * (dP[(int)rr] - del_s[ro + qr]) : 0.f;
          }
        });
        if constexpr (kBF) {
          bf16x8 pb[2], sb[2];
          static_for<2>([&](auto hh) {
            static_for<8>([&](auto e) { pb[hh][(int)e] = (bf16)S[8 * hh + e]; sb[hh][(int)e] = (bf16)dP[8 * hh + e]; });
          });
          static_for<2>([&](auto hh) {
            static_for<DP / 32>([&](auto db) {
              const bf16x8 bo = tr_operand<C::RS>(dOs, ro + 16 * hh, 32 * db, lane);
              const bf16x8 bq = tr_operand<C::RS>(Qs, ro + 16 * hh, 32 * db, lane);
              dV[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pb[hh], bo, dV[db], 0, 0, 0);
              dK[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sb[hh], bq, dK[db], 0, 0, 0);
            });
          });
        } else {
          static_for<16>([&](auto rr) {
            const int qr = ro + 8 * (rr >> 2) + 4 * g + (rr & 3);
            static_for<DP / 32>([&](auto db) {
              dV[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(S[(int)rr], dOTs[(32 * db + lr) * C::TS + qr], dV[db], 0, 0, 0);
              dK[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(dP[(int)rr], QTs[(32 * db + lr) * C::TS + qr], dK[db], 0, 0, 0);
            });
          });
        }
      });
      __syncthreads();                      // every wave is done with this fill
      if (nxt < f1) store_fill();
      __syncthreads();
      qf = nxt;
    }
  };
  auto store = [&](float* dk, float* dv) {
    if (kw0 >= a.Tp) return;
    static_for<DP / 32>([&](auto db) {
      static_for<16>([&](auto rr) {
        const int64_t off = (bh * a.Tp + kw0 + 8 * (rr >> 2) + 4 * g + (rr & 3)) * DP + 32 * db + lr;
        dk[off] = dK[db][(int)rr] * a.scale;
        dv[off] = dV[db][(int)rr];
      });
    });
  };
  if constexpr (WRAP) {
    const int64_t qhi = k0 + 128 < a.T ? k0 + 128 : a.T;          // queries before some key of the block
    sweep(a.qw, a.dow, a.qw_t, a.dow_t, 0, qhi, std::integral_constant<int, kRelWrap>{});
    store(a.dkw, a.dvw);
    sweep(a.qh, a.doh, a.qh_t, a.doh_t, k0, a.T, std::integral_constant<int, kRelBase>{});
  } else {
    sweep(a.qh, a.doh, a.qh_t, a.doh_t, 0, a.T, std::integral_constant<int, kRelAll>{});
  }
  store(a.dkh, a.dvh);
}

template <typename T, int DP, bool WRAP, bool DROP = false>
__global__ void __launch_bounds__(kBwdThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 2 : 1)))
attn_bwd_masked_dq(MaskedBwdArgs a) {
  using C = BwdCfg<T, DP>;
  typedef typename frag<T>::type frag_t;
  constexpr bool kBF = sizeof(T) == 2;
  using M = typename TileCopy<T, DP>::template Multi<2, kBF ? 0 : 1>;
  __shared__ __align__(16) T tiles[M::kElems];
  const T* const Ks = tiles;
  const T* const Vs = tiles + M::kRowTile;
  const T* const KTs = tiles + 2 * M::kRowTile;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t nqb = (a.Tp + 127) / 128;
  const int64_t qb = (int64_t)blockIdx.x / nbh, bh = blockIdx.x % nbh;
  const int64_t q0 = qb * 128, qw0 = q0 + 32 * w, q = qw0 + lr;
  const int64_t nw = a.Tp / 64;
  (void)nqb;

  frag_t qf[C::QF], df[C::QF];
  auto load_rows = [&](const void* qsrc, const void* dsrc) {
    const bool in = qw0 < a.Tp;
    const T* qrow = reinterpret_cast<const T*>(qsrc) + (bh * a.Tp + q) * DP;
    const T* drow = reinterpret_cast<const T*>(dsrc) + (bh * a.Tp + q) * DP;
    static_for<C::QF>([&](auto s) {
      if constexpr (kBF) {
        qf[s] = in ? *reinterpret_cast<const bf16x8*>(qrow + 16 * s + 8 * g) : bf16x8{};
        df[s] = in ? *reinterpret_cast<const bf16x8*>(drow + 16 * s + 8 * g) : bf16x8{};
      } else {
        qf[s] = in ? qrow[2 * s + g] : 0.f;
        df[s] = in ? drow[2 * s + g] : 0.f;
      }
    });
  };
  const bool qin = q < a.T;
  const float lse = qin ? a.lse[bh * a.Tp + q] : INFINITY;
  const float del = qin ? a.delta[bh * a.Tp + q] : 0.f;
  const float cl = a.scale_log2;
  f32x16 dQ[DP / 32];
  static_for<DP / 32>([&](auto i) { dQ[i] = f32x16{}; });

  // one branch over the key fills covering [klo, khi)
  auto sweep = [&](int64_t klo, int64_t khi, auto rel_c) {
    constexpr int rel = decltype(rel_c)::value;
    if (khi <= klo) return;
    const int f0 = (int)(klo / kFill), f1 = (int)((khi + kFill - 1) / kFill);
    for (int kfi = f0; kfi < f1; ++kfi) {
      const int64_t k0 = (int64_t)kfi * kFill;
      // a fill the mask closes for all of the workgroup's queries (the map of
      // open (128-query, 64-key) tiles; the same byte for every thread)
      if (a.tile_act != nullptr && a.tile_act[qb * nw + kfi] == 0) continue;
      {
        u32x4 r[M::IT];
        const T* const rows[2] = {reinterpret_cast<const T*>(a.kh) + (bh * a.Tp + k0) * DP,
                                  reinterpret_cast<const T*>(a.vh) + (bh * a.Tp + k0) * DP};
        const T* const cols[1] = {kBF ? nullptr : reinterpret_cast<const T*>(a.kh_t) + (bh * a.nch + k0 / kChunk) * DP * kChunk};
        M::load(r, rows, cols, 0, tid);
        __syncthreads();                    // the previous fill is consumed
        M::store(tiles, r, tid);
        __syncthreads();
      }
      // this lane's mask word over the fill's 64 keys (fills are 64-aligned)
      const uint64_t mw = a.mask_bits == nullptr ? ~0ull : (qin ? a.mask_bits[q * nw + k0 / 64] : 0ull);
      static_for<kFill / kBT>([&](auto sub) {
        const int64_t ks0 = k0 + kBT * sub;
        if (qw0 >= a.T) return;
        if (rel == kRelBase && ks0 > qw0 + kBT - 1) return;    // every key after every query
        if (rel == kRelWrap && ks0 + kBT - 1 <= qw0) return;   // no key after any query
        const int ro = kBT * sub;
        // a sub-tile whose 32 keys the mask closes for all of the wave's
        // queries adds only zeros: skip it (uniform over the wave)
        if (a.mask_bits != nullptr && !__any(((mw >> ro) & 0xffffffffull) != 0ull)) return;
        f32x16 S = f32x16{}, dP = f32x16{};
        static_for<C::QF>([&](auto s) {
          if constexpr (kBF) {
            const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&Ks[(ro + lr) * C::RS + 16 * s + 8 * g]);
            const bf16x8 va = *reinterpret_cast<const bf16x8*>(&Vs[(ro + lr) * C::RS + 16 * s + 8 * g]);
            S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], S, 0, 0, 0);
            dP = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, df[s], dP, 0, 0, 0);
          } else {
            S = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[(ro + lr) * C::RS + 2 * s + g], qf[s], S, 0, 0, 0);
            dP = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[(ro + lr) * C::RS + 2 * s + g], df[s], dP, 0, 0, 0);
          }
        });
        // dropout: elements 4 G .. 4 G + 3 are four consecutive keys of this
        // lane's query, the four words of one Philox call
        float z[DROP ? 16 : 1];
        if constexpr (DROP) {
          static_for<4>([&](auto G) {
            const u32x4 wd = keep_words(q, (k0 + ro + 8 * G + 4 * g) >> 2, bh, a.drop);
            static_for<4>([&](auto e) { z[4 * G + e] = wd[(int)e] >= a.drop.thr ? a.drop.scale : 0.f; });
          });
        }
        // element r: key ks0 + kr (row), this lane's query (column)
        static_for<16>([&](auto rr) {
          const int kr = ro + 8 * (rr >> 2) + 4 * g + (rr & 3);    // key offset in the fill
          const int64_t kk = k0 + kr;
          bool ok = kk < a.T && ((mw >> kr) & 1ull) != 0ull;
          if constexpr (rel == kRelBase) ok = ok && kk <= q;
          if constexpr (rel == kRelWrap) ok = ok && kk > q;
          const float pm = ok ? exp2f(__builtin_fmaf(S[(int)rr], cl, -lse)) : 0.f;
          if constexpr (DROP) dP[(int)rr] = ok ? pm * (z[(int)rr] * dP[(int)rr] - del) : 0.f;
          else dP[(int)rr] = ok ? pm * (dP[(int)rr] - del) : 0.f;
        });
        if constexpr (kBF) {
          bf16x8 sb[2];
          static_for<2>([&](auto hh) { static_for<8>([&](auto e) { sb[hh][(int)e] = (bf16)dP[8 * hh + e]; }); });
          static_for<2>([&](auto hh) {
            static_for<DP / 32>([&](auto db) {
              const bf16x8 av = tr_operand<C::RS>(Ks, ro + 16 * hh, 32 * db, lane);
              dQ[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, sb[hh], dQ[db], 0, 0, 0);
            });
          });
        } else {
          static_for<16>([&](auto rr) {
            const int kr = ro + 8 * (rr >> 2) + 4 * g + (rr & 3);
            static_for<DP / 32>([&](auto db) {
              dQ[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(KTs[(32 * db + lr) * C::TS + kr], dP[(int)rr], dQ[db], 0, 0, 0);
            });
          });
        }
      });
    }
  };
  auto store = [&](float* dq) {
    if (qw0 >= a.Tp) return;
    float* dst = dq + (bh * a.Tp + q) * DP;
    static_for<DP / 32>([&](auto db) {
      static_for<4>([&](auto r4) {
        f32x4 v;
        static_for<4>([&](auto i) { v[(int)i] = dQ[db][4 * r4 + i] * a.scale; });
        *reinterpret_cast<f32x4*>(&dst[32 * db + 8 * r4 + 4 * g]) = v;
      });
    });
  };
  const int64_t q_end = q0 + 128 < a.T ? q0 + 128 : a.T;          // one past the block's last query
  load_rows(a.qh, a.doh);
  if constexpr (WRAP) {
    sweep(0, q_end, std::integral_constant<int, kRelBase>{});
    store(a.dqh);
    static_for<DP / 32>([&](auto i) { dQ[i] = f32x16{}; });
    load_rows(a.qw, a.dow);
    sweep(q0, a.T, std::integral_constant<int, kRelWrap>{});
    store(a.dqw);
  } else {
    sweep(0, a.T, std::integral_constant<int, kRelAll>{});
    store(a.dqh);
  }
}

// The holonomy's cross sum (causal exact path): with dkw, dvw the wrap
// branch's dK^, dV^, Hol^T dL/dHol has the antisymmetric part of
//   c_hol = sum_j k^_j x dkw_j + v^_j x dvw_j   (per block),
// which link_bwd adds to every suffix (Hol is P_T of the link recursion).
// One workgroup per (b, h); fixed summation order.
template <typename T, int DP>
__global__ void __launch_bounds__(kBwdThreads) hol_torque(MaskedBwdArgs a) {
  constexpr int NBJ = (DP / 3 + 3) / 4;
  constexpr int NV = 3 * NBJ;
  __shared__ float part[4][4][NV];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t bh = blockIdx.x;
  const int tl = tid >> 2, p = tid & 3;
  const int blk0 = p * NBJ;
  const int nblk = a.nb - blk0 < 0 ? 0 : (a.nb - blk0 < NBJ ? a.nb - blk0 : NBJ);
  const int nd = 3 * nblk, e0 = 3 * blk0;
  float cv[NV];
  static_for<NV>([&](auto i) { cv[i] = 0.f; });
  for (int64_t t = tl; t < a.T; t += kChunk) {
    const int64_t row = (bh * a.Tp + t) * DP + e0;
    float x[NV], y[NV];
    auto add_cross = [&]() {
      static_for<NBJ>([&](auto j) {
        cv[3 * j] += x[3 * j + 1] * y[3 * j + 2] - x[3 * j + 2] * y[3 * j + 1];
        cv[3 * j + 1] += x[3 * j + 2] * y[3 * j] - x[3 * j] * y[3 * j + 2];
        cv[3 * j + 2] += x[3 * j] * y[3 * j + 1] - x[3 * j + 1] * y[3 * j];
      });
    };
    load_span<T, NV, false>(reinterpret_cast<const T*>(a.kh) + row, nd, x);
    load_span<float, NV, false>(a.dkw + row, nd, y);
    add_cross();
    load_span<T, NV, false>(reinterpret_cast<const T*>(a.vh) + row, nd, x);
    load_span<float, NV, false>(a.dvw + row, nd, y);
    add_cross();
  }
  // the wave's 16 tokens (lanes of equal p, stride 4), then the 4 waves
  static_for<4>([&](auto s) {
    constexpr int off = 32 >> s;
    static_for<NV>([&](auto i) {
      const float xs = __shfl_down(cv[i], off);
      if (lane + off < 64) cv[i] += xs;
    });
  });
  if (lane < 4) static_for<NV>([&](auto i) { part[w][lane][i] = cv[i]; });
  __syncthreads();
  if (tid < a.nb) {
    const int bp = tid / NBJ, bj = tid % NBJ;
    float* dst = a.hol_torque + (bh * a.nb + tid) * 4;
    static_for<3>([&](auto k) {
      dst[k] = ((part[0][bp][3 * bj + k] + part[1][bp][3 * bj + k]) + part[2][bp][3 * bj + k]) + part[3][bp][3 * bj + k];
    });
    dst[3] = 0.f;
  }
}

// The exact path's backward: (mask bits packed by the caller) prep, dK/dV,
// dQ, the holonomy's cross sum (causal), then the chained link kernel.
template <typename IO, typename GT, int DP, int EX>
static hipError_t launch_masked_bwd_ex(const MaskedBwdArgs& a, hipStream_t s) {
  constexpr bool WRAP = EX == 1;
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t nblk = (a.Tp + 127) / 128;
  const dim3 grid((unsigned)(nbh * nblk));
  hipLaunchKernelGGL((bwd_prep<IO, DP, EX>), dim3((unsigned)(nbh * a.nch)), dim3(kBwdThreads), 0, s, a);
  if (a.dropout) {
    hipLaunchKernelGGL((attn_bwd_masked_dkdv<IO, DP, WRAP, true>), grid, dim3(kBwdThreads), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_masked_dq<IO, DP, WRAP, true>), grid, dim3(kBwdThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_masked_dkdv<IO, DP, WRAP>), grid, dim3(kBwdThreads), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_masked_dq<IO, DP, WRAP>), grid, dim3(kBwdThreads), 0, s, a);
  }
  if constexpr (WRAP)
    hipLaunchKernelGGL((hol_torque<IO, DP>), dim3((unsigned)nbh), dim3(kBwdThreads), 0, s, a);
  hipError_t e = launch_chain_reset(a.carry, nbh * a.nch * a.nb * 2, a.ticket, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((link_bwd<IO, GT, DP, false, EX>), dim3((unsigned)(nbh * a.nch)), dim3(kBwdThreads), 0, s, a);
  return hipGetLastError();
}

template <typename IO, typename GT>
hipError_t launch_masked_bwd(const MaskedBwdArgs& a, hipStream_t s) {
  const bool causal = a.mode == 0;
  switch (a.Dp) {
    case 32: return causal ? launch_masked_bwd_ex<IO, GT, 32, 1>(a, s) : launch_masked_bwd_ex<IO, GT, 32, 2>(a, s);
    case 64: return causal ? launch_masked_bwd_ex<IO, GT, 64, 1>(a, s) : launch_masked_bwd_ex<IO, GT, 64, 2>(a, s);
    case 96: return causal ? launch_masked_bwd_ex<IO, GT, 96, 1>(a, s) : launch_masked_bwd_ex<IO, GT, 96, 2>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t launch_masked_bwd<float, float>(const MaskedBwdArgs&, hipStream_t);
template hipError_t launch_masked_bwd<bf16, float>(const MaskedBwdArgs&, hipStream_t);

// keep[(bh T + i) T + j] = 1 when attention dropout keeps pair (i, j) of
// head bh: one thread per (bh, i, j / 4), the four words of one Philox call
__global__ void __launch_bounds__(256) dropout_keep(int64_t nbh, int64_t T, DropParams d, uint8_t* keep) {
  const int64_t nj4 = (T + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= nbh * T * nj4) return;
  const int64_t j4 = idx % nj4, row = idx / nj4;           // row = bh T + i
  const int64_t i = row % T, bh = row / T;
  const u32x4 wd = keep_words(i, j4, bh, d);
  uint8_t* dst = keep + row * T + 4 * j4;
  static_for<4>([&](auto e) {
    if (4 * j4 + e < T) dst[(int)e] = wd[(int)e] >= d.thr ? 1 : 0;
  });
}

hipError_t launch_dropout_keep(int B, int H, int64_t T, const DropParams& d, uint8_t* keep, hipStream_t s) {
  const int64_t nbh = (int64_t)B * H, n = nbh * T * ((T + 3) / 4);
  if (n == 0) return hipSuccess;
  if ((n + 255) / 256 > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dropout_keep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, nbh, T, d, keep);
  return hipGetLastError();
}

}  // namespace holo
