// Kernel templates of the attention backward (holo_bwd.hip: the causal +
// tril path; holo_bwd_masked.hip: the exact path, any mask and either mode).
// The derivation and the kernel sequence are described in holo_bwd.hip.
#pragma once
#include <type_traits>

#include "holo_chain.h"
#include "holo_kernels.h"

namespace holo {

constexpr int kBT = 32;              // queries / keys per backward MFMA tile
constexpr int kFill = 64;            // rows per LDS fill of the dQ kernel (two MFMA tiles)
#ifndef HOLO_DKDV_FILL
#define HOLO_DKDV_FILL 32
#endif
constexpr int kFillKV = HOLO_DKDV_FILL;   // query rows per LDS fill of the dK/dV kernel
constexpr int kBwdThreads = 256;     // 4 waves

template <typename T, int DP, int ROWS = kFill> struct BwdCfg {
  static constexpr int E = 16 / sizeof(T);        // elements per 16 bytes
  static constexpr int RS = DP + E;               // LDS stride of a row-major tile row
  static constexpr int TS = ROWS + E;             // LDS stride of a transposed tile row (16 B aligned)
  static constexpr int QF = sizeof(T) == 2 ? DP / 16 : DP / 2;   // MFMA k-steps over DP
};

template <typename T> struct frag;
template <> struct frag<bf16> { typedef bf16x8 type; };
template <> struct frag<float> { typedef float type; };

// A 32x32x16 bf16 MFMA operand whose k index runs over the rows of a row-major
// LDS tile (row stride RS): lane l gets column col0 + l % 32 at rows
// row0 + 4 (l / 32) + {0..3} and row0 + 8 + 4 (l / 32) + {0..3}, the k order
// of an accumulator used as the other operand. ds_read_b64_tr_b16 hands lane i
// of each 16-lane group element i % 4 of the 4-element reads of lanes
// i / 4 + {0, 4, 8, 12}; source lane r of group G reads row
// row0 + 4 (G / 2) + r / 4, columns col0 + 16 (G % 2) + 4 (r % 4) + {0..3}, so
// lane i receives column col0 + 16 (G % 2) + i at four consecutive rows.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <int RS>
__device__ __forceinline__ bf16x8 tr_operand(const bf16* tile, int row0, int col0, int lane) {
  const int G = lane >> 4, r = lane & 15;
  const int row = row0 + 4 * (G >> 1) + (r >> 2), col = col0 + 16 * (G & 1) + 4 * (r & 3);
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + row * RS + col));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + (row + 8) * RS + col));
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), h4 = __builtin_bit_cast(bf16x4, hi);
  return bf16x8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
}

// Cooperative copies of ROWS-row / ROWS-column tiles into LDS. All of a
// thread's global loads are issued before its LDS stores (one memory round
// trip per tile, not one per chunk).
template <typename T, int DP, int ROWS = kFill> struct TileCopy {
  using C = BwdCfg<T, DP, ROWS>;
  static constexpr int RCPR = DP / C::E, TCPR = ROWS / C::E;   // 16-byte chunks per row
  static constexpr int RN = ROWS * RCPR, TN = DP * TCPR;        // chunks per tile
  // NA tiles at once, flattened over the threads: tile k's chunk i is flat
  // index k*RN + i (row-major tiles first, then transposed ones)
  template <int NR, int NT>
  struct Multi {
    static constexpr int N = NR * RN + NT * TN;
    static constexpr int IT = (N + kBwdThreads - 1) / kBwdThreads;
    static __device__ __forceinline__ void load(u32x4 (&r)[IT], const T* const (&rows)[NR], const T* const* cols,
                                                int j0, int tid) {
      static_for<IT>([&](auto it) {
        const int f = tid + kBwdThreads * it;
        if (f < NR * RN) {
          const int k = f / RN, i = f % RN;
          r[it] = *reinterpret_cast<const u32x4*>(&rows[k][(int64_t)(i / RCPR) * DP + (i % RCPR) * C::E]);
        } else if (f < N) {
          const int k = (f - NR * RN) / TN, i = (f - NR * RN) % TN;
          r[it] = *reinterpret_cast<const u32x4*>(&cols[k][(int64_t)(i / TCPR) * kChunk + j0 + (i % TCPR) * C::E]);
        }
      });
    }
    // LDS destination: the NR row-major tiles (ROWS * RS elements each), then
    // the NT transposed tiles (DP * TS each), back to back from `lds`
    static constexpr int kRowTile = ROWS * C::RS, kColTile = DP * C::TS;
    static constexpr int kElems = NR * kRowTile + NT * kColTile;
    static __device__ __forceinline__ void store(T* lds, const u32x4 (&r)[IT], int tid) {
      static_for<IT>([&](auto it) {
        const int f = tid + kBwdThreads * it;
        if (f < NR * RN) {
          const int k = f / RN, i = f % RN;
          *reinterpret_cast<u32x4*>(&lds[k * kRowTile + (i / RCPR) * C::RS + (i % RCPR) * C::E]) = r[it];
        } else if (f < N) {
          const int k = (f - NR * RN) / TN, i = (f - NR * RN) % TN;
          *reinterpret_cast<u32x4*>(&lds[NR * kRowTile + k * kColTile + (i / TCPR) * C::TS + (i % TCPR) * C::E]) = r[it];
        }
      });
    }
  };
};

// ---------------------------------------------------------------------------
// bwd_prep
// ---------------------------------------------------------------------------
// Transposes a 64 x DP row-major tile (src) into the (DP, 64) layout (dst),
// or back when kToRows, through LDS (stride DP + E / 64 + E).
template <typename T, int DP, bool kToRows>
__device__ inline void transpose_tile(T* lds, const T* src, T* dst, int tid) {
  constexpr int E = 16 / sizeof(T);
  constexpr int SR = kToRows ? kChunk + E : DP + E;          // LDS stride of the source layout
  constexpr int NR = kToRows ? DP : kChunk;                  // source rows
  constexpr int NC = kToRows ? kChunk : DP;                  // source columns
  __syncthreads();
  for (int i = tid; i < NR * (NC / E); i += kBwdThreads) {
    const int r = i / (NC / E), cc = i % (NC / E);
    *reinterpret_cast<u32x4*>(&lds[r * SR + cc * E]) = *reinterpret_cast<const u32x4*>(&src[(int64_t)r * NC + cc * E]);
  }
  __syncthreads();
  // destination: NC rows of NR elements; chunk (row c, part j) gathers column c
  for (int i = tid; i < NC * (NR / E); i += kBwdThreads) {
    const int c = i / (NR / E), j = i % (NR / E);
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
    static_for<E>([&](auto k) { e[k] = lds[(j * E + k) * SR + c]; });
    *reinterpret_cast<u32x4*>(&dst[(int64_t)c * NR + j * E]) = raw;
  }
}

// EX (the backward variant, BwdArgsOf): 0 and 1 write doh = P^T do, 2 (inert)
// doh' = P do; 1 also writes the wrap branch's operands qw = Hol^T qh and
// dow = Hol^T doh (and, fp32, their transposed tiles).
template <typename T, int DP, int EX = 0>
__global__ void __launch_bounds__(kBwdThreads) bwd_prep(typename BwdArgsOf<EX>::type a) {
  constexpr int E = 16 / sizeof(T);
  constexpr int LDSN = (DP + E) * kChunk > (kChunk + E) * DP ? (DP + E) * kChunk : (kChunk + E) * DP;
  __shared__ float Ds[kChunk][DP + 1];
  __shared__ __align__(16) T Ts[LDSN];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x / a.nch, c = blockIdx.x % a.nch;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int tl = tid >> 2, p = tid & 3;
  const int64_t t = c * kChunk + tl;
  const bool in = t < a.T;

  // doh = P^T do and the row dot do . o (4 threads per token)
  for (int k = p; k < DP; k += 4) Ds[tl][k] = 0.f;
  __syncthreads();
  float dot = 0.f;
  const T* orow = reinterpret_cast<const T*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs;
  const T* drow = reinterpret_cast<const T*>(a.dout) + (b * a.T + t) * a.do_rs + h * a.do_hs;
  // d = 96 with 16-byte aligned rows: thread p owns dims [24p, 24p + 24) (8
  // whole blocks), read as 16-byte vectors, and its 8 quaternions (contiguous)
  const bool wide = DP == 96 && a.d == 96 &&
                    ((reinterpret_cast<uintptr_t>(drow) | reinterpret_cast<uintptr_t>(orow)) & 15) == 0;
  if (in && wide) {
    constexpr int E = 16 / sizeof(T);
    float u[24], v[24];
    static_for<24 / E>([&](auto cc) {
      const u32x4 ru = reinterpret_cast<const u32x4*>(drow + 24 * p)[cc];
      const u32x4 rv = reinterpret_cast<const u32x4*>(orow + 24 * p)[cc];
      const T* eu = reinterpret_cast<const T*>(&ru);
      const T* ev = reinterpret_cast<const T*>(&rv);
      static_for<E>([&](auto j) { u[cc * E + j] = to_f32(eu[j]); v[cc * E + j] = to_f32(ev[j]); });
    });
    const float* pq = a.P + ((bh * a.T + t) * a.nb + 8 * p) * 4;
    static_for<8>([&](auto jb) {
      const rot3 R = qmat(load_quat(pq + 4 * jb));
      dot += u[3 * jb] * v[3 * jb] + u[3 * jb + 1] * v[3 * jb + 1] + u[3 * jb + 2] * v[3 * jb + 2];
      float y0, y1, y2;
      if constexpr (EX == 2) rot_apply(R, u[3 * jb], u[3 * jb + 1], u[3 * jb + 2], y0, y1, y2);
      else rot_t_apply(R, u[3 * jb], u[3 * jb + 1], u[3 * jb + 2], y0, y1, y2);
      Ds[tl][24 * p + 3 * jb] = y0; Ds[tl][24 * p + 3 * jb + 1] = y1; Ds[tl][24 * p + 3 * jb + 2] = y2;
    });
  } else if (in) {
    for (int blk = p; blk < a.nb; blk += 4) {
      const rot3 R = qmat(load_quat(a.P + ((bh * a.T + t) * a.nb + blk) * 4));
      float u[3], v[3];
      static_for<3>([&](auto k) { u[k] = to_f32(drow[3 * blk + k]); v[k] = to_f32(orow[3 * blk + k]); });
      dot += u[0] * v[0] + u[1] * v[1] + u[2] * v[2];
      float y0, y1, y2;
      if constexpr (EX == 2) rot_apply(R, u[0], u[1], u[2], y0, y1, y2);
      else rot_t_apply(R, u[0], u[1], u[2], y0, y1, y2);
      Ds[tl][3 * blk] = y0; Ds[tl][3 * blk + 1] = y1; Ds[tl][3 * blk + 2] = y2;
    }
    if (p == 0) {
      for (int k = 3 * a.nb; k < a.d; ++k) {
        const float u = to_f32(drow[k]);
        dot += u * to_f32(orow[k]);
        Ds[tl][k] = u;
      }
    }
  }
  dot += __shfl_xor(dot, 1);
  dot += __shfl_xor(dot, 2);
  if (p == 0) a.delta[bh * a.Tp + t] = in ? dot : 0.f;
  __syncthreads();
  // doh rows and doh transposed tile
  T* dohr = reinterpret_cast<T*>(a.doh) + (bh * a.Tp + c * kChunk) * DP;
  for (int i = tid; i < kChunk * (DP / E); i += kBwdThreads) {
    const int r = i / (DP / E), cc = i % (DP / E);
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
    static_for<E>([&](auto k) { e[k] = from_f32<T>(Ds[r][cc * E + k]); });
    *reinterpret_cast<u32x4*>(&dohr[(int64_t)r * DP + cc * E]) = raw;
  }
  const int64_t row0 = (bh * a.Tp + c * kChunk) * DP, tile0 = (bh * a.nch + c) * DP * kChunk;
  if constexpr (sizeof(T) == 4) {
    // fp32 MFMA operands read the transposed layouts doh_t, qh_t, kh_t (bf16
    // reads them from the row-major tiles with transposing LDS reads)
    T* doht = reinterpret_cast<T*>(a.doh_t) + (bh * a.nch + c) * DP * kChunk;
    for (int i = tid; i < DP * (kChunk / E); i += kBwdThreads) {
      const int r = i / (kChunk / E), cc = i % (kChunk / E);
      u32x4 raw;
      T* e = reinterpret_cast<T*>(&raw);
      static_for<E>([&](auto k) { e[k] = from_f32<T>(Ds[cc * E + k][r]); });
      *reinterpret_cast<u32x4*>(&doht[(int64_t)r * kChunk + cc * E]) = raw;
    }
    transpose_tile<T, DP, false>(Ts, reinterpret_cast<const T*>(a.qh) + row0, reinterpret_cast<T*>(a.qh_t) + tile0, tid);
    transpose_tile<T, DP, false>(Ts, reinterpret_cast<const T*>(a.kh) + row0, reinterpret_cast<T*>(a.kh_t) + tile0, tid);
  }
  // vh row-major from the forward's transposed tiles
  transpose_tile<T, DP, true>(Ts, reinterpret_cast<const T*>(a.vh_t) + tile0, reinterpret_cast<T*>(a.vh) + row0, tid);
  if constexpr (EX == 1) {
    // the rows in Ds (fp32) to a row-major destination and, fp32, its
    // transposed tile
    auto put_rows = [&](void* rows, void* cols) {
      T* dr = reinterpret_cast<T*>(rows) + row0;
      for (int i = tid; i < kChunk * (DP / E); i += kBwdThreads) {
        const int r = i / (DP / E), cc = i % (DP / E);
        u32x4 raw;
        T* e = reinterpret_cast<T*>(&raw);
        static_for<E>([&](auto k) { e[k] = from_f32<T>(Ds[r][cc * E + k]); });
        *reinterpret_cast<u32x4*>(&dr[(int64_t)r * DP + cc * E]) = raw;
      }
      if constexpr (sizeof(T) == 4) {
        T* dt = reinterpret_cast<T*>(cols) + tile0;
        for (int i = tid; i < DP * (kChunk / E); i += kBwdThreads) {
          const int r = i / (kChunk / E), cc = i % (kChunk / E);
          u32x4 raw;
          T* e = reinterpret_cast<T*>(&raw);
          static_for<E>([&](auto k) { e[k] = from_f32<T>(Ds[cc * E + k][r]); });
          *reinterpret_cast<u32x4*>(&dt[(int64_t)r * kChunk + cc * E]) = raw;
        }
      }
    };
    // the blocks of every row of Ds rotated by Hol^T in place
    auto hol_t_rows = [&]() {
      for (int i = tid; i < kChunk * a.nb; i += kBwdThreads) {
        const int r = i / a.nb, blk = i % a.nb;
        const rot3 R = qmat(load_quat(a.hol + (bh * a.nb + blk) * 4));
        float y0, y1, y2;
        rot_t_apply(R, Ds[r][3 * blk], Ds[r][3 * blk + 1], Ds[r][3 * blk + 2], y0, y1, y2);
        Ds[r][3 * blk] = y0; Ds[r][3 * blk + 1] = y1; Ds[r][3 * blk + 2] = y2;
      }
    };
    __syncthreads();                       // Ds holds doh; every earlier read of it is done
    hol_t_rows();
    __syncthreads();
    put_rows(a.dow, a.dow_t);
    __syncthreads();
    const T* qr = reinterpret_cast<const T*>(a.qh) + row0;
    for (int i = tid; i < kChunk * DP; i += kBwdThreads) Ds[i / DP][i % DP] = to_f32(qr[i]);
    __syncthreads();
    hol_t_rows();
    __syncthreads();
    put_rows(a.qw, a.qw_t);
  }
}

// ---------------------------------------------------------------------------
// attention backward: dK, dV
// ---------------------------------------------------------------------------
// MFMA register layouts (32x32 tiles): the A operand lane l holds row l % 32,
// the B operand column l % 32, each 8 (bf16) or 1 (fp32) values of the k
// range; the accumulator lane l holds column l % 32 and rows
// 8 (r / 4) + 4 (l / 32) + (r % 4), r = 0..15. A product whose k index runs
// over the accumulator rows of an earlier product uses that same order for
// both operands, so the accumulator is the operand with no data movement.
template <typename T, int DP>
__global__ void __launch_bounds__(kBwdThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 2 : 1))) attn_bwd_dkdv(BwdArgs a) {
  using C = BwdCfg<T, DP, kFillKV>;
  typedef typename frag<T>::type frag_t;
  constexpr bool kBF = sizeof(T) == 2;
  // Q and dO row-major; fp32 also loads the transposed tiles Q^T, dO^T (bf16
  // reads the transposed operands from the row-major tiles, tr_operand)
  using M = typename TileCopy<T, DP, kFillKV>::template Multi<2, kBF ? 0 : 2>;
  __shared__ __align__(16) T tiles[M::kElems];
  __shared__ float lse_s[kFillKV], del_s[kFillKV];
  __shared__ __align__(16) T Kw[128 * C::RS];      // the workgroup's 128 key rows (B operand of S = Q K^T)
  const T* const Qs = tiles;
  const T* const dOs = tiles + M::kRowTile;
  const T* const QTs = tiles + 2 * M::kRowTile;
  const T* const dOTs = tiles + 2 * M::kRowTile + M::kColTile;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t kb = blockIdx.x / nbh, bh = blockIdx.x % nbh;      // key block 0 (most queries) first
  const int64_t k0 = kb * 128, kw0 = k0 + 32 * w;
  const bool wave_in = kw0 < a.T;

  // this wave's 32 keys: V rows as B operands in registers (key = lane % 32),
  // the K rows of all 128 keys in LDS
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
  const int nfill = (int)((a.T + kFillKV - 1) / kFillKV);
  const int qf0 = (int)(k0 / kFillKV);
  // fill qf+1 is loaded into registers while fill qf is computed from LDS
  u32x4 r[M::IT];
  float ls = INFINITY, dl = 0.f;
  auto load_fill = [&](int qf) {
    const int64_t q0 = (int64_t)qf * kFillKV;
    const int64_t tile = (bh * a.nch + q0 / kChunk) * DP * kChunk;
    const T* const rows[2] = {reinterpret_cast<const T*>(a.qh) + (bh * a.Tp + q0) * DP,
                              reinterpret_cast<const T*>(a.doh) + (bh * a.Tp + q0) * DP};
    const T* const cols[2] = {kBF ? nullptr : reinterpret_cast<const T*>(a.qh_t) + tile,
                              kBF ? nullptr : reinterpret_cast<const T*>(a.doh_t) + tile};
    M::load(r, rows, cols, (int)(q0 % kChunk), tid);
    const bool qin = tid < kFillKV && q0 + tid < a.T;
    ls = qin ? a.lse[bh * a.Tp + q0 + tid] : INFINITY;
    dl = qin ? a.delta[bh * a.Tp + q0 + tid] : 0.f;
  };
  auto store_fill = [&]() {
    M::store(tiles, r, tid);
    if (tid < kFillKV) { lse_s[tid] = ls; del_s[tid] = dl; }
  };
  if (qf0 < nfill) { load_fill(qf0); store_fill(); }
  __syncthreads();
  for (int qf = qf0; qf < nfill; ++qf) {
    const int64_t q0 = (int64_t)qf * kFillKV;
    if (qf + 1 < nfill) load_fill(qf + 1);
    static_for<kFillKV / kBT>([&](auto sub) {
      const int64_t qs0 = q0 + kBT * sub;
      if (!wave_in || qs0 + kBT - 1 < kw0) return;    // no query of the tile sees these keys
      const int ro = kBT * sub;                       // row offset of the tile within the fill

      // S = Q K^T and dP = dO V^T (queries on the rows, this wave's keys on the lanes)
      f32x16 S = f32x16{}, dP = f32x16{};
      static_for<C::QF>([&](auto s) {
        if constexpr (kBF) {
          const bf16x8 qa = *reinterpret_cast<const bf16x8*>(&Qs[(ro + lr) * C::RS + 16 * s + 8 * g]);
          const bf16x8 da = *reinterpret_cast<const bf16x8*>(&dOs[(ro + lr) * C::RS + 16 * s + 8 * g]);
          const bf16x8 kb = *reinterpret_cast<const bf16x8*>(&Kw[(32 * w + lr) * C::RS + 16 * s + 8 * g]);
          S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kb, S, 0, 0, 0);
          dP = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vf[s], dP, 0, 0, 0);
        } else {
          S = __builtin_amdgcn_mfma_f32_32x32x2f32(Qs[(ro + lr) * C::RS + 2 * s + g], Kw[(32 * w + lr) * C::RS + 2 * s + g], S, 0, 0, 0);
          dP = __builtin_amdgcn_mfma_f32_32x32x2f32(dOs[(ro + lr) * C::RS + 2 * s + g], vf[s], dP, 0, 0, 0);
        }
      });
      // Pm = exp2(scale_log2 S - lse) (zero above the diagonal and for padding
      // keys; padding queries carry lse = +inf), dS = Pm (dP - delta)
      static_for<16>([&](auto r) {
        const int qr = 8 * (r >> 2) + 4 * g + (r & 3);
        float pm = exp2f(__builtin_fmaf(S[(int)r], cl, -lse_s[ro + qr]));
        if (key > qs0 + qr || key >= a.T) pm = 0.f;
        S[(int)r] = pm;
        dP[(int)r] = pm * (dP[(int)r] - del_s[ro + qr]);
      });
      // dV += Pm^T dO, dK += dS^T Q (this wave's keys on the rows, dims on the lanes)
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
        static_for<16>([&](auto r) {
          const int qr = ro + 8 * (r >> 2) + 4 * g + (r & 3);
          static_for<DP / 32>([&](auto db) {
            dV[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(S[(int)r], dOTs[(32 * db + lr) * C::TS + qr], dV[db], 0, 0, 0);
            dK[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(dP[(int)r], QTs[(32 * db + lr) * C::TS + qr], dK[db], 0, 0, 0);
          });
        });
      }
    });
    __syncthreads();                        // every wave is done with this fill
    if (qf + 1 < nfill) store_fill();
    __syncthreads();
  }
  if (kw0 < a.Tp) {
    static_for<DP / 32>([&](auto db) {
      static_for<16>([&](auto r) {
        const int64_t off = (bh * a.Tp + kw0 + 8 * (r >> 2) + 4 * g + (r & 3)) * DP + 32 * db + lr;
        a.dkh[off] = dK[db][(int)r] * a.scale;
        a.dvh[off] = dV[db][(int)r];
      });
    });
  }
}

// ---------------------------------------------------------------------------
// attention backward: dQ
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ void __launch_bounds__(kBwdThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 2 : 1))) attn_bwd_dq(BwdArgs a) {
  using C = BwdCfg<T, DP>;
  typedef typename frag<T>::type frag_t;
  constexpr bool kBF = sizeof(T) == 2;
  // K and V row-major; fp32 also loads K^T (bf16 reads it from K, tr_operand)
  using M = typename TileCopy<T, DP>::template Multi<2, kBF ? 0 : 1>;
  __shared__ __align__(16) T tiles[M::kElems];
  const T* const Ks = tiles;
  const T* const Vs = tiles + M::kRowTile;
  const T* const KTs = tiles + 2 * M::kRowTile;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t nqb = (a.Tp + 127) / 128;
  const int64_t qb = nqb - 1 - (int64_t)blockIdx.x / nbh, bh = blockIdx.x % nbh;   // longest first
  const int64_t q0 = qb * 128, qw0 = q0 + 32 * w, q = qw0 + lr;

  // this wave's 32 queries: Q and dO rows as B operands (query = lane % 32)
  frag_t qf[C::QF], df[C::QF];
  {
    const bool in = qw0 < a.Tp;
    const T* qrow = reinterpret_cast<const T*>(a.qh) + (bh * a.Tp + q) * DP;
    const T* drow = reinterpret_cast<const T*>(a.doh) + (bh * a.Tp + q) * DP;
    static_for<C::QF>([&](auto s) {
      if constexpr (kBF) {
        qf[s] = in ? *reinterpret_cast<const bf16x8*>(qrow + 16 * s + 8 * g) : bf16x8{};
        df[s] = in ? *reinterpret_cast<const bf16x8*>(drow + 16 * s + 8 * g) : bf16x8{};
      } else {
        qf[s] = in ? qrow[2 * s + g] : 0.f;
        df[s] = in ? drow[2 * s + g] : 0.f;
      }
    });
  }
  const bool qin = q < a.T;
  const float lse = qin ? a.lse[bh * a.Tp + q] : INFINITY;
  const float del = qin ? a.delta[bh * a.Tp + q] : 0.f;
  const float cl = a.scale_log2;
  f32x16 dQ[DP / 32];
  static_for<DP / 32>([&](auto i) { dQ[i] = f32x16{}; });

  int64_t qlast = q0 + 127 < a.T - 1 ? q0 + 127 : a.T - 1;    // the workgroup's last query
  const int nfill = qlast >= q0 ? (int)(qlast / kFill) + 1 : 0;
  for (int kfi = 0; kfi < nfill; ++kfi) {
    const int64_t k0 = (int64_t)kfi * kFill;
    {
      u32x4 r[M::IT];
      const T* const rows[2] = {reinterpret_cast<const T*>(a.kh) + (bh * a.Tp + k0) * DP,
                                reinterpret_cast<const T*>(a.vh) + (bh * a.Tp + k0) * DP};
      const T* const cols[1] = {kBF ? nullptr : reinterpret_cast<const T*>(a.kh_t) + (bh * a.nch + k0 / kChunk) * DP * kChunk};
      M::load(r, rows, cols, 0, tid);
      __syncthreads();                      // the previous fill is consumed
      M::store(tiles, r, tid);
      __syncthreads();
    }
    static_for<kFill / kBT>([&](auto sub) {
      const int64_t ks0 = k0 + kBT * sub;
      if (qw0 >= a.T || ks0 > qw0 + kBT - 1) return;     // every key of the tile is after every query
      const int ro = kBT * sub;

      // S^T = K Q^T and dP^T = V dO^T (keys on the rows, this wave's queries on the lanes)
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
      static_for<16>([&](auto r) {
        const int64_t kr = ks0 + 8 * (r >> 2) + 4 * g + (r & 3);
        float pm = exp2f(__builtin_fmaf(S[(int)r], cl, -lse));
        if (kr > q || kr >= a.T) pm = 0.f;
        dP[(int)r] = pm * (dP[(int)r] - del);
      });
      // dQ^T += K^T dS^T (dims on the rows, queries on the lanes)
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
        static_for<16>([&](auto r) {
          const int kr = ro + 8 * (r >> 2) + 4 * g + (r & 3);
          static_for<DP / 32>([&](auto db) {
            dQ[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(KTs[(32 * db + lr) * C::TS + kr], dP[(int)r], dQ[db], 0, 0, 0);
          });
        });
      }
    });
  }
  if (qw0 < a.Tp) {
    float* dst = a.dqh + (bh * a.Tp + q) * DP;
    static_for<DP / 32>([&](auto db) {
      static_for<4>([&](auto r4) {
        f32x4 v;
        static_for<4>([&](auto i) { v[(int)i] = dQ[db][4 * r4 + i] * a.scale; });
        *reinterpret_cast<f32x4*>(&dst[32 * db + 8 * r4 + 4 * g]) = v;
      });
    });
  }
}

// ---------------------------------------------------------------------------
// link_bwd: suffix scan of the per-token cross products, link gradients,
// and dq, dk, dv in the reference frame
// ---------------------------------------------------------------------------
// dL/da for a = (a01, a02, a12) of one block from g = vee(W - W^T),
// W = G^T dL/dG: a is phi = (-a12, a02, -a01) in the standard hat map and
// dL/dphi = J_r(phi)^T g = g + al phi x g + be phi x (phi x g),
// al = (1 - cos th)/th^2 = 2 sin^2(th/2)/th^2, be = (th - sin th)/th^3
// (Taylor series of be below th = 1, where the closed form cancels).
__device__ inline void link_param_grad(float a0, float a1, float a2, const float (&gv)[3], float (&da)[3]) {
  const float ph[3] = {-a2, a1, -a0};
  const float th2 = ph[0] * ph[0] + ph[1] * ph[1] + ph[2] * ph[2];
  float al, be;
  if (th2 < 1.f) {
    al = 0.5f + th2 * (-1.f / 24.f + th2 * (1.f / 720.f - th2 * (1.f / 40320.f)));
    be = 1.f / 6.f + th2 * (-1.f / 120.f + th2 * (1.f / 5040.f - th2 * (1.f / 362880.f)));
  } else {
    const float th = sqrtf(th2);
    float sh, ch;
    sincosf(0.5f * th, &sh, &ch);
    al = 2.f * sh * sh / th2;
    be = (th - 2.f * sh * ch) / (th2 * th);
  }
  float pxg[3] = {ph[1] * gv[2] - ph[2] * gv[1], ph[2] * gv[0] - ph[0] * gv[2], ph[0] * gv[1] - ph[1] * gv[0]};
  float ppg[3] = {ph[1] * pxg[2] - ph[2] * pxg[1], ph[2] * pxg[0] - ph[0] * pxg[2], ph[0] * pxg[1] - ph[1] * pxg[0]};
  float dph[3];
  static_for<3>([&](auto k) { dph[k] = gv[k] + al * pxg[k] + be * ppg[k]; });
  da[0] = -dph[2];
  da[1] = dph[1];
  da[2] = -dph[0];
}

// N contiguous elements of one row as fp32: 16-byte vector accesses on the
// wide path (rows and spans 16-byte aligned), element accesses otherwise;
// `n` (<= N) elements are valid.
template <typename T, int N, bool WIDE>
__device__ __forceinline__ void load_span(const T* p, int n, float (&v)[N]) {
  constexpr int E = 16 / sizeof(T);
  if constexpr (WIDE && N % E == 0) {
    static_for<N / E>([&](auto c) {
      const u32x4 raw = reinterpret_cast<const u32x4*>(p)[c];
      const T* e = reinterpret_cast<const T*>(&raw);
      static_for<E>([&](auto i) { v[c * E + i] = to_f32(e[i]); });
    });
  } else {
    static_for<N>([&](auto i) { v[i] = i < n ? to_f32(p[i]) : 0.f; });
  }
}

template <typename T, int N, bool WIDE>
__device__ __forceinline__ void store_span(T* p, int n, const float (&v)[N]) {
  constexpr int E = 16 / sizeof(T);
  if constexpr (WIDE && N % E == 0) {
    static_for<N / E>([&](auto c) {
      u32x4 raw;
      T* e = reinterpret_cast<T*>(&raw);
      static_for<E>([&](auto i) { e[i] = from_f32<T>(v[c * E + i]); });
      reinterpret_cast<u32x4*>(p)[c] = raw;
    });
  } else {
    static_for<N>([&](auto i) { if (i < n) p[i] = from_f32<T>(v[i]); });
  }
}

// Thread (token tl = tid / 4, part p = tid % 4) owns blocks p*NBJ .. p*NBJ+NBJ-1
// of its token: 3*NBJ contiguous dims of every row it reads or writes.
// EX (BwdArgsOf): 1, the causal exact path, adds the wrap branch's dQ (Hol
// dqw) to dqh and starts the suffix from the holonomy's cross sum (the
// virtual token T = Hol), which also gives the closing edge its gradient;
// 2, inert mode, reads primed values (u' = P u): the cross sums c' of that
// frame give c = -P^T c' and the gradients return by P^T.
template <typename IO, typename GT, int DP, bool WIDE, int EX = 0>
__global__ void __launch_bounds__(kBwdThreads) link_bwd(typename BwdArgsOf<EX>::type a) {
  constexpr int NBJ = (DP / 3 + 3) / 4;          // blocks per thread
  constexpr int NV = 3 * NBJ;                    // dims per thread
  __shared__ float wtot[4][4][NV];               // [wave][p][dim]: the wave's inclusive suffix at its first token
  __shared__ float carry[DP];                     // suffix sum of all later chunks, per (block, component)
  __shared__ unsigned s_ticket;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) s_ticket = __hip_atomic_fetch_add(a.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int64_t nbh = (int64_t)a.B * a.H, tk = s_ticket;
  if (tk / nbh >= a.nch) return;                  // only if the counter was not reset
  const int64_t c = a.nch - 1 - tk / nbh, bh = tk % nbh;   // last chunk first
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int tl = tid >> 2, p = tid & 3;
  const int64_t t = c * kChunk + tl;
  const bool in = t < a.T;
  const int blk0 = p * NBJ;
  const int nblk = a.nb - blk0 < 0 ? 0 : (a.nb - blk0 < NBJ ? a.nb - blk0 : NBJ);   // valid blocks
  const int nd = 3 * nblk, e0 = 3 * blk0;

  quat qP[NBJ];
  float cv[NV];
  static_for<NV>([&](auto i) { cv[i] = 0.f; });
  const int64_t prow = (bh * a.Tp + t) * DP + e0;
  if (in) {
    const float* pq = a.P + ((bh * a.T + t) * a.nb + blk0) * 4;
    static_for<NBJ>([&](auto j) { qP[j] = j < nblk ? load_quat(pq + 4 * j) : qident(); });
    // c_t = oh x doh + dqh x qh + dkh x kh + dvh x vh per block
    float u[NV], v[NV];
    load_span<IO, NV, WIDE>(reinterpret_cast<const IO*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs + e0, nd, u);
    load_span<IO, NV, WIDE>(reinterpret_cast<const IO*>(a.dout) + (b * a.T + t) * a.do_rs + h * a.do_hs + e0, nd, v);
    static_for<NBJ>([&](auto j) {
      const rot3 R = qmat(qP[j]);
      float oh[3], dh[3];
      if constexpr (EX == 2) {
        rot_apply(R, u[3 * j], u[3 * j + 1], u[3 * j + 2], oh[0], oh[1], oh[2]);
        rot_apply(R, v[3 * j], v[3 * j + 1], v[3 * j + 2], dh[0], dh[1], dh[2]);
      } else {
        rot_t_apply(R, u[3 * j], u[3 * j + 1], u[3 * j + 2], oh[0], oh[1], oh[2]);
        rot_t_apply(R, v[3 * j], v[3 * j + 1], v[3 * j + 2], dh[0], dh[1], dh[2]);
      }
      cv[3 * j] += oh[1] * dh[2] - oh[2] * dh[1];
      cv[3 * j + 1] += oh[2] * dh[0] - oh[0] * dh[2];
      cv[3 * j + 2] += oh[0] * dh[1] - oh[1] * dh[0];
    });
    // cv += grad x value, and the gradient rotated back to the reference
    // frame (dq = P dqh, ...) while it is in registers
    auto acc = [&](const void* gsrc, const float* src, void* dst, int64_t rs, int64_t hs, const float* wsrc) {
      load_span<IO, NV, WIDE>(reinterpret_cast<const IO*>(gsrc) + prow, nd, v);
      load_span<float, NV, WIDE>(src + prow, nd, u);
      if constexpr (EX == 1) {
        if (wsrc != nullptr) {              // + Hol dqw: the wrap branch's dQ in the path frame
          float x[NV];
          load_span<float, NV, WIDE>(wsrc + prow, nd, x);
          static_for<NBJ>([&](auto j) {
            if (j < nblk) {
              float y0, y1, y2;
              rot_apply(qmat(load_quat(a.hol + (bh * a.nb + blk0 + j) * 4)), x[3 * j], x[3 * j + 1], x[3 * j + 2],
                        y0, y1, y2);
              u[3 * j] += y0; u[3 * j + 1] += y1; u[3 * j + 2] += y2;
            }
          });
        }
      }
      static_for<NBJ>([&](auto j) {
        cv[3 * j] += u[3 * j + 1] * v[3 * j + 2] - u[3 * j + 2] * v[3 * j + 1];
        cv[3 * j + 1] += u[3 * j + 2] * v[3 * j] - u[3 * j] * v[3 * j + 2];
        cv[3 * j + 2] += u[3 * j] * v[3 * j + 1] - u[3 * j + 1] * v[3 * j];
      });
      static_for<NBJ>([&](auto j) {
        if constexpr (EX == 2)
          rot_t_apply(qmat(qP[j]), u[3 * j], u[3 * j + 1], u[3 * j + 2], v[3 * j], v[3 * j + 1], v[3 * j + 2]);
        else
          rot_apply(qmat(qP[j]), u[3 * j], u[3 * j + 1], u[3 * j + 2], v[3 * j], v[3 * j + 1], v[3 * j + 2]);
      });
      store_span<IO, NV, WIDE>(reinterpret_cast<IO*>(dst) + (b * a.T + t) * rs + h * hs + e0, nd, v);
    };
    const float* dqw = nullptr;
    if constexpr (EX == 1) dqw = a.dqw;
    acc(a.qh, a.dqh, a.dq, a.dq_rs, a.dq_hs, dqw);
    acc(a.kh, a.dkh, a.dk, a.dk_rs, a.dk_hs, nullptr);
    acc(a.vh, a.dvh, a.dv, a.dv_rs, a.dv_hs, nullptr);
    if constexpr (EX == 2) {               // c = -P^T c'
      static_for<NBJ>([&](auto j) {
        float y0, y1, y2;
        rot_t_apply(qmat(qP[j]), cv[3 * j], cv[3 * j + 1], cv[3 * j + 2], y0, y1, y2);
        cv[3 * j] = -y0; cv[3 * j + 1] = -y1; cv[3 * j + 2] = -y2;
      });
    }
  }
  // inclusive suffix over the wave's 16 tokens (lane + 4 is the next token)
  float sv[NV];
  static_for<NV>([&](auto i) { sv[i] = cv[i]; });
  static_for<4>([&](auto s) {
    constexpr int off = 4 << s;
    static_for<NV>([&](auto i) {
      const float x = __shfl_down(sv[i], off);
      if (lane + off < 64) sv[i] += x;
    });
  });
  if (lane < 4) static_for<NV>([&](auto i) { wtot[w][p][i] = sv[i]; });
  __syncthreads();
  // chained carry: chunk c publishes (its total) + (the suffix of chunks > c)
  if (tid < a.nb) {
    const int blk = tid, bp = blk / NBJ, bj = blk % NBJ;
    float tot[3];
    static_for<3>([&](auto k) {
      tot[k] = ((wtot[0][bp][3 * bj + k] + wtot[1][bp][3 * bj + k]) + wtot[2][bp][3 * bj + k]) + wtot[3][bp][3 * bj + k];
    });
    quat nxt = quat{0.f, 0.f, 0.f, 0.f};
    if (c + 1 < a.nch) {
      const float* slot = a.carry + ((bh * a.nch + c + 1) * a.nb + blk) * 4;
      bool ok = false;
      for (int polls = 0; polls < kMaxPolls; ++polls) {
        if (get_quat(slot, nxt)) { ok = true; break; }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!ok) {
        __hip_atomic_fetch_or(a.ticket + 1, kStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float nan = __uint_as_float(kCanonNan);
        nxt = quat{nan, nan, nan, nan};
      }
    }
    if constexpr (EX == 1) {
      if (c + 1 == a.nch) {                 // the last chunk starts from the holonomy's cross sum
        const float* ht = a.hol_torque + (bh * a.nb + blk) * 4;
        nxt = quat{ht[0], ht[1], ht[2], 0.f};
      }
    }
    if (c > 0)
      put_quat(a.carry + ((bh * a.nch + c) * a.nb + blk) * 4, quat{nxt.w + tot[0], nxt.x + tot[1], nxt.y + tot[2], 0.f});
    carry[3 * blk] = nxt.w; carry[3 * blk + 1] = nxt.x; carry[3 * blk + 2] = nxt.y;
  }
  __syncthreads();
  if (!in) return;

  // m_{t+1} = (suffix within the chunk, tokens > t) + later waves + later chunks;
  // dL/da_t from P_t m_{t+1} (the closing edge's m is zero, no later tokens,
  // unless the holonomy's cross sum seeded the last chunk's carry)
  const int64_t tn = t + 1 == a.T ? 0 : t + 1;
  float ga[NV], da[NV];
  load_span<GT, NV, WIDE>(reinterpret_cast<const GT*>(a.gq) + (b * a.T + t) * a.gq_rs + h * a.gq_hs + e0, nd, ga);
  if (a.gen_mode == 0) {
    float gk[NV];
    load_span<GT, NV, WIDE>(reinterpret_cast<const GT*>(a.gk) + (b * a.T + tn) * a.gk_rs + h * a.gk_hs + e0, nd, gk);
    static_for<NV>([&](auto i) { ga[i] += gk[i]; });
  }
  static_for<NBJ>([&](auto j) {
    float m[3];
    static_for<3>([&](auto k) {
      float later = 0.f;
      for (int w2 = w + 1; w2 < 4; ++w2) later += wtot[w2][p][3 * j + k];
      m[k] = (sv[3 * j + k] - cv[3 * j + k]) + later + (j < nblk ? carry[e0 + 3 * j + k] : 0.f);
    });
    float gv[3], d3[3];
    rot_apply(qmat(qP[j]), m[0], m[1], m[2], gv[0], gv[1], gv[2]);
    link_param_grad(a.edge_scale * ga[3 * j], a.edge_scale * ga[3 * j + 1], a.edge_scale * ga[3 * j + 2], gv, d3);
    static_for<3>([&](auto k) { da[3 * j + k] = a.edge_scale * d3[k]; });
  });
  store_span<float, NV, WIDE>(a.dgq + (b * a.T + t) * a.dgq_rs + h * a.dgq_hs + e0, nd, da);
  if (a.gen_mode == 0) store_span<float, NV, WIDE>(a.dgk + (b * a.T + tn) * a.dgk_rs + h * a.dgk_hs + e0, nd, da);
  if (p == 0) {
    const int64_t prow0 = (bh * a.Tp + t) * DP;
    for (int e = 3 * a.nb; e < a.d; ++e) {     // dims outside the rotation blocks
      float dqe = a.dqh[prow0 + e];
      if constexpr (EX == 1) dqe += a.dqw[prow0 + e];
      reinterpret_cast<IO*>(a.dq)[(b * a.T + t) * a.dq_rs + h * a.dq_hs + e] = from_f32<IO>(dqe);
      reinterpret_cast<IO*>(a.dk)[(b * a.T + t) * a.dk_rs + h * a.dk_hs + e] = from_f32<IO>(a.dkh[prow0 + e]);
      reinterpret_cast<IO*>(a.dv)[(b * a.T + t) * a.dv_rs + h * a.dv_hs + e] = from_f32<IO>(a.dvh[prow0 + e]);
    }
  }
}

}  // namespace holo
