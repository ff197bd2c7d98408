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
// Work decomposition: one workgroup (4 waves) per (b, h) and folded pair of
// 128-query tiles (a long and a short tile, run one after the other); each
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
// The queries arrive already transported (qh from the scan); the back-rotation
// o_i = P_i oh_i is fused into the epilogue, which stages the tile's outputs
// through LDS and rotates each 3-dim block by its stored quaternion.
// Two kernels share this decomposition and the epilogue: attn_fwd_h16 (16-bit
// operands, bf16 or fp16, on the MFMA; three waves per SIMD, tile loads that
// write LDS directly) and attn_fwd (fp32 MFMA, two waves per SIMD,
// register-staged tile loads). The output o is written in its own type OT:
// the operand type's companion (bf16 for the bf16 path) or fp32.
#include <type_traits>

#include "holo_attn_common.h"

namespace holo {

// Epilogue of a 128-query tile: normalise the wave's O^T accumulator (dims on
// the MFMA rows, its 32 queries on the lanes) by the row sums, stage it in LDS
// (fp32 rows of OS), then back-rotate o = P oh per 3-dim block with the stored
// quaternions (int16 or fp32) and write 16-byte rows of o in type T. Os may
// alias the key/value ring: every read of the ring must be complete.
template <typename T, int DP, bool PQ16>
__device__ __forceinline__ void store_tile_output(const AttnArgs& a, float* Os, const f32x16 (&O)[DP / 32],
                                                  float m_run, float l_run, int64_t q0, int64_t qw, int bh,
                                                  int b, int h, int tid, int w, int lr, int g) {
  using C = AttnCfg<float, DP>;                  // staging layout (fp32 rows of OS)
  const float lt = pair_sum(l_run);
  const float inv = __builtin_amdgcn_rcpf(fmaxf(lt, 1e-20f));
  if (a.lse && g == 0 && qw + lr < a.T) a.lse[(int64_t)bh * a.Tp + qw + lr] = m_run + __log2f(lt);
  // items (row, 8 consecutive 3-dim groups = 24 dims); a row's 8 quaternions
  // are 128 contiguous bytes in fp32, 64 in int16. Their loads are issued
  // before the staging (the loop's registers are free by then: O and the
  // quaternions fit), so the staging and its barrier cover their latency.
  typedef typename std::conditional<PQ16, u32x2, f32x4>::type pq_t;
  const pq_t pq_ident = [] {
    if constexpr (PQ16) return u32x2{1u, 0u};            // (1, 0, 0, 0)
    else return f32x4{1.f, 0.f, 0.f, 0.f};
  }();
  pq_t pq[C::EPI][8];
  static_for<C::EPI>([&](auto it) {
    const int idx = tid + it * kThreads, r = idx / C::NG8, gi = idx % C::NG8;
    const int64_t t = q0 + r;
    const bool row_ok = idx < kBM * C::NG8 && t < a.T;
    const pq_t* base = reinterpret_cast<const pq_t*>(
        reinterpret_cast<const char*>(a.P) + ((bh * a.T + t) * a.nb + 8 * gi) * (int64_t)sizeof(pq_t));
    if (row_ok && 8 * gi + 8 <= a.nb) {
      static_for<8>([&](auto jb) { pq[it][jb] = base[jb]; });
    } else {
      static_for<8>([&](auto jb) { pq[it][jb] = (row_ok && 8 * gi + jb < a.nb) ? base[jb] : pq_ident; });
    }
  });
  static_for<DP / 32>([&](auto db) {
    static_for<16>([&](auto r) {
      Os[(32 * w + lr) * C::OS + 32 * db + 8 * (r >> 2) + 4 * g + (r & 3)] = O[db][(int)r] * inv;
    });
  });
  __syncthreads();
  // item = (row, 8 consecutive 3-dim groups = 24 dims), quaternions in pq
  static_for<C::EPI>([&](auto it) {
    const int idx = tid + it * kThreads, r = idx / C::NG8, gi = idx % C::NG8;
    const int64_t t = q0 + r;
    if (idx >= kBM * C::NG8 || t >= a.T || 24 * gi >= a.d) return;
    float u[24];
    static_for<24>([&](auto j) { u[j] = (24 * gi + j < DP) ? Os[r * C::OS + 24 * gi + j] : 0.f; });
    static_for<8>([&](auto jb) {
      if (8 * gi + jb < a.nb) {
        float y0, y1, y2;
        quat qr;
        if constexpr (PQ16) qr = unpack_quat_snorm16(pq[it][jb]);
        else qr = quat{pq[it][jb][0], pq[it][jb][1], pq[it][jb][2], pq[it][jb][3]};
        quat_rotate(qr, u[3 * jb], u[3 * jb + 1], u[3 * jb + 2], y0, y1, y2);
        u[3 * jb] = y0; u[3 * jb + 1] = y1; u[3 * jb + 2] = y2;
      }
    });
    T* orow = reinterpret_cast<T*>(a.o) + (b * a.T + t) * a.o_rs + h * a.o_hs + 24 * gi;
    if (24 * gi + 24 <= a.d && (reinterpret_cast<uintptr_t>(orow) & 15) == 0) {
      constexpr int E = 16 / sizeof(T);
      static_for<24 / E>([&](auto cc) {
        u32x4 raw;
        T* e = reinterpret_cast<T*>(&raw);
        static_for<E>([&](auto j) { e[j] = from_f32<T>(u[cc * E + j]); });
        reinterpret_cast<u32x4*>(orow)[cc] = raw;
      });
    } else {
      static_for<24>([&](auto j) {
        if (24 * gi + j < a.d) orow[j] = from_f32<T>(u[j]);
      });
    }
  });
}

// fp32 kernel (mfma_f32_32x32x2f32). Pipeline over key tiles j = 0, 1, ...:
// three LDS stages hold tiles j, j+1 and j+2; registers hold tile j+3 in flight. Iteration j issues the QK MFMAs
// of tile j+1, then runs the softmax and PV MFMAs of tile j (so the VALU work
// overlaps the matrix core), stores tile j+2 into the free stage, issues the
// loads of tile j+3 and ends with the tile's only barrier.
template <typename T, int DP, bool PQ16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
attn_fwd(AttnArgs a) {
  static_assert(sizeof(T) == 4, "16-bit operands run attn_fwd_h16");
  using C = AttnCfg<T, DP>;
  extern __shared__ __align__(16) unsigned char smem[];
  T* const kv = reinterpret_cast<T*>(smem);
  float* const Os = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int lr = lane & 31;               // query column of this lane (MFMA col)
  const int g = lane >> 5;                // lane half
  // Causal query tiles differ in length, so each workgroup runs a folded pair
  // of one (b, h): query tile ntile-1-f, then tile f (alone when they
  // coincide). Every pair of tiles covers ntile+1 key tiles of 128 keys, so
  // all workgroups carry the same work and the grid ends without a tail.
  // Workgroup L runs on XCD L % 8; when B*H is a multiple of 8, XCD x takes the
  // (b, h) pairs congruent to x and runs the folds of one pair back to back, so
  // a pair's keys/values stay in that XCD's L2.
  const int ntile = (int)((a.T + kBM - 1) / kBM);
  const int nfold = (ntile + 1) / 2;
  const int L = blockIdx.x;
  int bh, f;
  if ((a.B * a.H) % 8 == 0) {
    const int j = L >> 3;
    bh = 8 * (j / nfold) + (L & 7);
    f = j % nfold;
  } else {
    bh = L % (a.B * a.H);
    f = L / (a.B * a.H);
  }
  const int b = bh / a.H, h = bh % a.H;
  auto run_tile = [&](const int qt) {
    const int64_t q0 = (int64_t)qt * kBM;
    const int64_t qw = q0 + 32 * w;                       // first query of this wave

    // ---- Q^T operand straight from qh (the scan's transported queries) ----
    constexpr int QF = DP / 2;                            // Q^T operand steps
    float qf[QF];
    {
      const int64_t qrow_t = qw + lr;                     // rows past Tp read as zero
      const T* qrow = reinterpret_cast<const T*>(a.qh) + ((int64_t)bh * a.Tp + qrow_t) * DP;
      const bool in = qrow_t < a.Tp;
      static_for<QF>([&](auto s) { qf[s] = in ? qrow[2 * s + g] : 0.f; });
    }

    f32x16 O[DP / 32];
    static_for<DP / 32>([&](auto i) { O[i] = f32x16{}; });
    float m_run = -1e30f, l_run = 0.f;
    const float c = a.scale_log2;

    int64_t kend = q0 + kBM; if (kend > a.T) kend = a.T;
    const int nkv = (int)((kend + kBN - 1) / kBN);
    // tiles this wave attends to: keys up to its last query (0 when past T)
    const int nact = qw >= a.T ? 0 : (int)((qw + 31) / kBN) + 1 < nkv ? (int)((qw + 31) / kBN) + 1 : nkv;
    const u32x4* kbase = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.kh) + (int64_t)bh * a.Tp * DP);
    const u32x4* vbase = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.vh_t) + (int64_t)bh * a.nch * DP * kBN);
    constexpr int TCH = kBN * DP / C::E;                  // 16 B chunks per tile
    constexpr int RC = DP / C::E, VC = kBN / C::E;        // chunks per K row / V^T row

    u32x4 kreg[C::KCH], vreg[C::VCH];
    // buffer loads: the (b, h) slice in a scalar resource descriptor, the tile
    // offset in a scalar register and a constant byte offset per lane, so a
    // tile load costs no per-lane address arithmetic
    const int kv_bytes = (int)((int64_t)a.Tp * DP * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(kbase), 0, kv_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(vbase), 0, kv_bytes, kBufferWord3);
    auto load_tile = [&](int kt) {
      const int toff = kt * TCH * 16;
      static_for<C::KCH>([&](auto j) {
        kreg[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, (tid + j * kThreads) * 16, toff, 0);
      });
      static_for<C::VCH>([&](auto j) {
        vreg[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (tid + j * kThreads) * 16, toff, 0);
      });
    };
    auto store_tile = [&](int st) {
      T* Ks = kv + st * C::kStage;
      T* Vs = Ks + kBN * C::KS;
      static_for<C::KCH>([&](auto j) {
        int i = tid + j * kThreads, r = i / RC, cc = i % RC;
        *reinterpret_cast<u32x4*>(&Ks[r * C::KS + cc * C::E]) = kreg[j];
      });
      static_for<C::VCH>([&](auto j) {
        int i = tid + j * kThreads, r = i / VC, cc = i % VC;
        u32x2* dst = reinterpret_cast<u32x2*>(&Vs[r * C::VS + cc * C::E]);
        dst[0] = vreg[j].xy;
        dst[1] = vreg[j].zw;
      });
    };
    // S^T (64 keys x 32 queries) of the tile in stage st
    auto qk = [&](int st, f32x16 (&S)[2]) {
      const T* Ks = kv + st * C::kStage;
      S[0] = f32x16{}; S[1] = f32x16{};
      static_for<QF>([&](auto s) {
        static_for<2>([&](auto kb) {
          const float av = Ks[(32 * kb + lr) * C::KS + 2 * s + g];
          S[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, qf[s], S[kb], 0, 0, 0);
        });
      });
    };
    // online softmax (log2 units, one lane pair per query) and O^T += V^T P^T
    // of tile kt (stage st); the QK MFMAs of the next tile (stage stn, into Sn)
    // are issued in the same basic block as the exponentials so the two overlap.
    auto softmax_pv = [&](int kt, int st, f32x16 (&S)[2], int stn, f32x16 (&Sn)[2]) {
      const T* Vs = kv + st * C::kStage + kBN * C::KS;
      const int64_t k0 = (int64_t)kt * kBN;
      if (k0 + kBN - 1 > qw) {             // tile reaches past this wave's first query
        const int rel = (int)(qw - k0) + lr - 4 * g;     // key offset limit for this lane
        static_for<2>([&](auto kb) {
          static_for<16>([&](auto r) {
            if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) S[kb][(int)r] = -INFINITY;
          });
        });
      }
      const float mx = pair_max(tile_max(S)) * c;
      // each row decides for itself (a row's result never depends on its
      // neighbours'); the wave-uniform branch only skips the work, rare after warm-up
      const bool need = mx > m_run + kRescaleThreshold;
      if (__any(need)) {
        const float m_new = need ? mx : m_run;
        const float corr = exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= corr;
        static_for<DP / 32>([&](auto i) { O[i] *= corr; });
      }
      const float nm = -m_run;
      qk(stn, Sn);
      static_for<2>([&](auto kb) {
        static_for<16>([&](auto r) { S[kb][(int)r] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kb][(int)r], c, nm)); });
      });
      float t[16];
      static_for<16>([&](auto r) { t[r] = S[0][(int)r] + S[1][(int)r]; });
      static_for<8>([&](auto r) { t[r] += t[r + 8]; });
      static_for<4>([&](auto r) { t[r] += t[r + 4]; });
      static_for<2>([&](auto r) { t[r] += t[r + 2]; });
      l_run += t[0] + t[1];
      static_for<2>([&](auto kb) {
        static_for<16>([&](auto r) {
          static_for<DP / 32>([&](auto db) {
            float av = Vs[(32 * db + lr) * C::VS + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3)];
            O[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, S[kb][(int)r], O[db], 0, 0, 0);
          });
        });
      });
    };
    // one pipeline step: tile j in S, tile j+1 into Sn
    auto step = [&](int j, f32x16 (&S)[2], f32x16 (&Sn)[2]) {
      // (the next tile's QK runs whenever this tile does; past the wave's last
      // tile its result is never used)
      if (j < nact) softmax_pv(j, j % 3, S, (j + 1) % 3, Sn);
      if (j + 2 < nkv) store_tile((j + 2) % 3);
      if (j + 3 < nkv) load_tile(j + 3);
      __syncthreads();
    };

    // ---- fill: tiles 0 and 1 into stages 0 and 1, tile 2 into registers ----
    load_tile(0);
    store_tile(0);
    if (nkv > 1) { load_tile(1); store_tile(1); }
    if (nkv > 2) load_tile(2);
    __syncthreads();
    f32x16 SA[2], SB[2];
    if (nact > 0) qk(0, SA);
    for (int j = 0; j < nkv; j += 2) {
      step(j, SA, SB);
      if (j + 1 < nkv) step(j + 1, SB, SA);
    }
    store_tile_output<T, DP, PQ16>(a, Os, O, m_run, l_run, q0, qw, bh, b, h, tid, w, lr, g);
  };
  run_tile(ntile - 1 - f);
  if (f != ntile - 1 - f) {
    __syncthreads();                       // the first tile's epilogue is done with the LDS
    run_tile(f);
  }
}

// ---------------------------------------------------------------------------
// 16-bit kernel (operands OPT = bf16 or fp16, output OT): three waves per
// SIMD. The same work decomposition (folded pairs
// of 128-query tiles, 4 waves x 32 queries, 64-key tiles), built to fit three
// workgroups per CU so that a third wave per SIMD hides the latency that two
// leave exposed (dependent MFMA results, LDS reads, barriers):
//   - key/value tiles reach LDS by buffer loads that write LDS directly
//     (buffer_load_dwordx4 ... lds) into a 2-stage ring: no staging registers
//     and no ds_write; tiles are stored unpadded with an XOR swizzle of their
//     16-byte chunks (k_swz, v_swz) under which the fragment reads are free of
//     bank conflicts; LDS 51.2 KB per workgroup (the epilogue's fp32 staging);
//   - one S buffer: the QK of tile j+1 is issued after the tile barrier and
//     the other waves on the SIMD overlap their softmax with it (<= 168 VGPRs:
//     160 at d = 96, no spills).
// Key order inside S^T: lane lr reads K row pi(lr) of each 32-key block (pi
// swaps the 4-row groups 1 and 2 of every 16), so register r of the S^T
// accumulator of lane (lr, g) holds key 16(r>>3) + 8g + (r&7): the P^T operand
// of one PV MFMA covers 8 consecutive keys, which is one 16-byte V^T chunk.
// Step j (stage j&1 holds tile j; tile j+1 is in flight to the other stage):
// softmax and PV of tile j; wait for this thread's loads; barrier; loads of
// tile j+2 into stage j&1; QK of tile j+1.
template <int DP> struct RingCfg {
  static constexpr int NCK = DP / 8;                        // 16-byte chunks per K row
  static constexpr int QF = DP / 16, NDB = DP / 32;
  static constexpr int KT = kBN * DP;                       // elements per K (= V^T) tile
  static constexpr int kTileBytes = KT * 2;
  static constexpr int kVRegion = 2 * kTileBytes;           // LDS: [K stage 0, 1][V stage 0, 1]
  static constexpr int NKB = NCK % 8 == 0 ? NCK / 2 : 2;    // per-lane K read bases
  static constexpr int NI = KT / 8 / kThreads;              // 16-byte loads per thread per K (V) tile
  static constexpr size_t kv_bytes = (size_t)4 * kTileBytes;
  static constexpr size_t lds = kv_bytes > AttnCfg<bf16, DP>::o_bytes ? kv_bytes : AttnCfg<bf16, DP>::o_bytes;
  static_assert(NI * 8 * kThreads == KT, "tile split");
};

// chunk XOR of K row r (NCK chunks per row); only the low four bits of r
// enter, so a lane's XOR is the same in every 32-row block
template <int NCK> __device__ __forceinline__ int k_swz(int r) {
  if constexpr (NCK % 8 == 0) return ((r >> 1) ^ ((r & 1) << 1)) & 7;
  else return ((r >> 2) ^ ((r >> 1) & 1)) & 3;
}
// chunk XOR of V^T row r (8 chunks per row); low five bits only
__device__ __forceinline__ int v_swz(int r) { return ((r & 7) ^ ((r >> 3) & 3)) & 7; }

template <typename OPT, typename OT, int DP, bool PQ16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
attn_fwd_h16(AttnArgs a) {
  using C = RingCfg<DP>;
  using T = OPT;
  using Op = Op16<OPT>;
  using v8 = typename Op::v8;
  using v2 = typename Op::v2;
  extern __shared__ __align__(16) unsigned char smem[];
  float* const Os = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ntile = (int)((a.T + kBM - 1) / kBM);
  const int nfold = (ntile + 1) / 2;
  const int L = blockIdx.x;
  int bh, f;                                  // folded pairs and XCD mapping as attn_fwd
  if ((a.B * a.H) % 8 == 0) {
    const int j = L >> 3;
    bh = 8 * (j / nfold) + (L & 7);
    f = j % nfold;
  } else {
    bh = L % (a.B * a.H);
    f = L / (a.B * a.H);
  }
  const int b = bh / a.H, h = bh % a.H;
  const T* kbase = reinterpret_cast<const T*>(a.kh) + (int64_t)bh * a.Tp * DP;
  const T* vbase = reinterpret_cast<const T*>(a.vh_t) + (int64_t)bh * a.nch * DP * kBN;

  // loads to LDS: 16-byte chunk p = i*256 + tid of a tile lands at LDS chunk p;
  // the lane fetches the (row, chunk) that the swizzle stores there
  int koff[C::NI], voff[C::NI];
  static_for<C::NI>([&](auto i) {
    const int p = i * kThreads + tid;
    const int rk = p / C::NCK, ck = (p % C::NCK) ^ k_swz<C::NCK>(rk);
    koff[i] = (rk * DP + ck * 8) * (int)sizeof(T);           // bytes
    const int rv = p >> 3, cv = (p & 7) ^ v_swz(rv);
    voff[i] = (rv * kBN + cv * 8) * (int)sizeof(T);
  });
  // buffer loads to LDS: the (b, h) slice in a buffer resource (reads past it
  // return zero), the tile offset in a scalar register and one 32-bit byte
  // offset per lane and load (a 64-bit global address per load would hold
  // twice the registers)
  const int kv_bytes = (int)((int64_t)a.Tp * DP * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kbase), 0, kv_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vbase), 0, kv_bytes, kBufferWord3);
  auto issue_tile = [&](int kt, auto st) {
    const int toff = kt * C::kTileBytes;
    unsigned char* ks = smem + decltype(st)::value * C::kTileBytes;
    unsigned char* vs = smem + C::kVRegion + decltype(st)::value * C::kTileBytes;
    static_for<C::NI>([&](auto i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(ks + (i * kThreads + 64 * w) * 16), 16, koff[i], toff, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(vs + (i * kThreads + 64 * w) * 16), 16, voff[i], toff, 0, 0);
    });
  };
  // fragment reads: a few per-lane base offsets plus compile-time offsets. K
  // chunk (2s+g)^kx: with a 2-bit XOR it is 4(s>>1) + ((2(s&1)+g)^kx), so two
  // bases cover every s; with a 3-bit XOR there is one base per s. V chunk
  // (4kb+2hh+g)^vx: one base per (kb, hh); db adds 32 rows.
  const int pr = (lr & ~12) | ((lr & 4) << 1) | ((lr & 8) >> 1);     // pi(lr)
  const int kx = k_swz<C::NCK>(pr), vx = v_swz(lr);
  int kb_off[C::NKB], vb_off[4];
  static_for<C::NKB>([&](auto i) { kb_off[i] = (pr * C::NCK + ((2 * i + g) ^ kx)) * 16; });
  static_for<4>([&](auto i) { vb_off[i] = C::kVRegion + (lr * 8 + ((2 * i + g) ^ vx)) * 16; });
  auto k_frag = [&](auto st, auto kb, auto s) -> v8 {
    constexpr int sv = decltype(s)::value;
    constexpr int bi = C::NCK % 8 == 0 ? sv : (sv & 1);
    constexpr int imm = decltype(st)::value * C::kTileBytes + decltype(kb)::value * 32 * C::NCK * 16 +
                        (C::NCK % 8 == 0 ? 0 : (sv >> 1) * 64);
    return *reinterpret_cast<const v8*>(smem + kb_off[bi] + imm);
  };
  auto v_frag = [&](auto st, auto kb, auto hh, auto db) -> v8 {
    constexpr int bi = 2 * decltype(kb)::value + decltype(hh)::value;
    constexpr int imm = decltype(st)::value * C::kTileBytes + decltype(db)::value * 32 * 8 * 16;
    return *reinterpret_cast<const v8*>(smem + vb_off[bi] + imm);
  };

  auto run_tile = [&](const int qt) {
    const int64_t q0 = (int64_t)qt * kBM;
    const int64_t qw = q0 + 32 * w;
    v8 qf[C::QF];                             // Q^T operand straight from qh
    {
      const int64_t qrow_t = qw + lr;         // rows past Tp read as zero
      const T* qrow = reinterpret_cast<const T*>(a.qh) + ((int64_t)bh * a.Tp + qrow_t) * DP;
      const bool in = qrow_t < a.Tp;
      static_for<C::QF>([&](auto s) { qf[s] = in ? *reinterpret_cast<const v8*>(qrow + 16 * s + 8 * g) : v8{}; });
    }
    f32x16 O[C::NDB];
    static_for<C::NDB>([&](auto i) { O[i] = f32x16{}; });
    float m_run = -1e30f, l_run = 0.f;
    const float c = a.scale_log2;
    int64_t kend = q0 + kBM; if (kend > a.T) kend = a.T;
    const int nkv = (int)((kend + kBN - 1) / kBN);
    const int nact = qw >= a.T ? 0 : (int)((qw + 31) / kBN) + 1 < nkv ? (int)((qw + 31) / kBN) + 1 : nkv;

    f32x16 S[2];
    auto qk = [&](auto st) {
      S[0] = f32x16{}; S[1] = f32x16{};
      static_for<C::QF>([&](auto s) {
        static_for<2>([&](auto kb) {
          S[kb] = Op::mfma(k_frag(st, kb, s), qf[s], S[kb]);
        });
      });
    };
    // online softmax (log2 units, one lane pair per query) and O^T += V^T P^T
    auto softmax_pv = [&](int kt, auto st) {
      const int64_t k0 = (int64_t)kt * kBN;
      if (k0 + kBN - 1 > qw) {                // tile reaches past this wave's first query
        const int rel = (int)(qw - k0) + lr - 8 * g;
        static_for<2>([&](auto kb) {
          static_for<16>([&](auto r) {
            if (32 * kb + 16 * (r >> 3) + (r & 7) > rel) S[kb][(int)r] = -INFINITY;
          });
        });
      }
      const float mx = pair_max(tile_max(S)) * c;
      const bool need = mx > m_run + kRescaleThreshold;     // per row; the branch only skips work
      if (__any(need)) {
        const float m_new = need ? mx : m_run;
        const float corr = exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= corr;
        static_for<C::NDB>([&](auto i) { O[i] *= corr; });
      }
      const float nm = -m_run;
      // P^T operands in the operand type; the row sum is taken over the same
      // rounded values
      v8 pb[2][2];
      const v2 one2 = {(T)1.f, (T)1.f};
      float ls[2][2];
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          static_for<8>([&](auto e) {
            pb[kb][hh][(int)e] = (T)__builtin_amdgcn_exp2f(__builtin_fmaf(S[kb][8 * hh + e], c, nm));
          });
          ls[kb][hh] = 0.f;
          static_for<4>([&](auto e) {
            v2 pr2 = {pb[kb][hh][2 * e], pb[kb][hh][2 * e + 1]};
            ls[kb][hh] = Op::dot2(pr2, one2, ls[kb][hh]);
          });
        });
      });
      l_run += (ls[0][0] + ls[0][1]) + (ls[1][0] + ls[1][1]);
      static_for<2>([&](auto kb) {
        static_for<2>([&](auto hh) {
          static_for<C::NDB>([&](auto db) {
            O[db] = Op::mfma(v_frag(st, kb, hh, db), pb[kb][hh], O[db]);
          });
        });
      });
    };
    auto step = [&](int j, auto st) {
      using SN = std::integral_constant<int, 1 - decltype(st)::value>;
      if (j < nact) softmax_pv(j, st);
      wait_vmem<0>();                         // this thread's loads of tile j+1
      ring_barrier();                         // every wave's loads landed, tile j read
      if (j + 2 < nkv) issue_tile(j + 2, st);
      if (j + 1 < nact) qk(SN{});
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    issue_tile(0, S0{});
    if (nkv > 1) { issue_tile(1, S1{}); wait_vmem<2 * C::NI>(); } else { wait_vmem<0>(); }
    ring_barrier();
    if (nact > 0) qk(S0{});
    for (int j = 0; j < nkv; j += 2) {
      step(j, S0{});
      if (j + 1 < nkv) step(j + 1, S1{});
    }
    // the last step's barrier follows every read of the ring and no load is
    // in flight, so the staging may overwrite it
    store_tile_output<OT, DP, PQ16>(a, Os, O, m_run, l_run, q0, qw, bh, b, h, tid, w, lr, g);
  };
  run_tile(ntile - 1 - f);
  if (f != ntile - 1 - f) {
    __syncthreads();                          // the first tile's epilogue is done with the LDS
    run_tile(f);
  }
}

template <typename T, typename OT, int DP, bool PQ16>
static hipError_t launch_attn_dp(const AttnArgs& a, hipStream_t s) {
  const int64_t nfold = ((a.T + kBM - 1) / kBM + 1) / 2;
  const dim3 grid((unsigned)(a.B * a.H * nfold));
  if constexpr (sizeof(T) == 2) {
    using C = RingCfg<DP>;
    static_assert(C::lds <= kMaxDynamicLds, "tile configuration exceeds the LDS of a workgroup");
    const hipError_t attr = allow_dynamic_lds<&attn_fwd_h16<T, OT, DP, PQ16>>();
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((attn_fwd_h16<T, OT, DP, PQ16>), grid, dim3(kThreads), C::lds, s, a);
  } else {
    static_assert(std::is_same<OT, float>::value, "the fp32 kernel writes fp32");
    using C = AttnCfg<T, DP>;
    static_assert(C::lds <= kMaxDynamicLds, "tile configuration exceeds the LDS of a workgroup");
    const hipError_t attr = allow_dynamic_lds<&attn_fwd<T, DP, PQ16>>();
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((attn_fwd<T, DP, PQ16>), grid, dim3(kThreads), C::lds, s, a);
  }
  return hipGetLastError();
}

template <typename T, typename OT, bool PQ16>
static hipError_t launch_attn_pf(const AttnArgs& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_attn_dp<T, OT, 32, PQ16>(a, s);
    case 64: return launch_attn_dp<T, OT, 64, PQ16>(a, s);
    case 96: return launch_attn_dp<T, OT, 96, PQ16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename OPT, typename OT>
hipError_t launch_attn(const AttnArgs& a, hipStream_t s) {
  return a.p_format ? launch_attn_pf<OPT, OT, true>(a, s) : launch_attn_pf<OPT, OT, false>(a, s);
}

template hipError_t launch_attn<float, float>(const AttnArgs&, hipStream_t);
template hipError_t launch_attn<bf16, bf16>(const AttnArgs&, hipStream_t);
template hipError_t launch_attn<bf16, float>(const AttnArgs&, hipStream_t);
template hipError_t launch_attn<f16, bf16>(const AttnArgs&, hipStream_t);
template hipError_t launch_attn<f16, float>(const AttnArgs&, hipStream_t);

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
      const int e = 3 * (r - 3 * br) + (c - 3 * bc);
#pragma unroll
      for (int k = 0; k < 9; ++k)
        if (k == e) val = R.m[k / 3][k % 3];
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
