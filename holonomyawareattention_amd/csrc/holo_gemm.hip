// Projections of the layer on gfx950 MFMA: one GEMM for the per-head
// interleaved q/k/v columns and the additive link generator.
//
// Reference behaviour (core/attention_fast_chunked.py):
//   qkv = x W_qkv^T                                   :69-71 (bf16 out here)
//   g_t = gq(x_t) + gk(x_{(t+1) mod T})               :80-84 (before edge_scale)
// The generator output never exists in two halves: its tiles run a second
// K segment over the token rows shifted by one position (wrapping inside each
// sequence of T tokens), so one accumulator holds x_t W_gq^T + x_{t+1} W_gk^T
// and the epilogue writes g_t in fp32 (384 bytes per token and head at
// d = 96, read once by the scan).
//
// Tiling (the launched form, launch_qkvg): 256 features x 256 tokens per
// workgroup, 8 waves of 64 x 128 on v_mfma_f32_32x32x16_bf16 (the weights on
// the MFMA rows, the tokens on the lanes, so a lane holds 4 consecutive
// features of one token per register quad). K advances in steps of 64
// through a 2-stage LDS ring (128 KB) filled by buffer loads that write LDS
// directly (no staging registers); tiles are stored unpadded with the 16-byte
// chunk c of row r at c ^ gemm_swz(r), under which the fragment reads of a
// wave are free of bank conflicts on gfx950 (measured). Step i waits for its
// own tile, meets the barrier (every wave has then finished step i-1, so its
// stage is free) and issues the loads of step i+1 into that stage before its
// 32 MFMAs per wave. The epilogue goes through LDS so that global stores are
// whole 16-byte pieces of token rows.
// Generator tiles do twice the work of q/k/v tiles and come first in the
// grid; each XCD takes a contiguous range of M-blocks, in groups of 8 that
// stay in its L2 while the N-blocks sweep the weights.
//
// The same kernel, by a compile-time mode, serves the interaction
// generator's edge MLP (core/attention_fast_chunked.py:56-60,73-76):
//   hid = GELU([x_t ; x_{t+1}] W1^T + b1)    the shifted-row K segment is the
//                                             pair's second half (MODE 1)
//   g   = hid W2^T                            one K segment, fp32 (MODE 2)
// MODE 0 is the projection GEMM above and compiles to the same instructions
// as before the modes existed.
#include "holo_attn_common.h"

namespace holo {

namespace {

// physical 16-byte chunk of logical chunk c in tile row r (rows of BK bf16):
// XOR with bits of r chosen so that each ds_read_b128 of a fragment (32 rows,
// two chunks) is free of bank conflicts (measured on gfx950); with BK = 32
// rows r and r + 32 take the same XOR, with BK = 64 it follows the parity of
// the 32-row block (two per-lane offsets per substep)
template <int BK> __device__ __forceinline__ int gemm_swz(int r) {
  if constexpr (BK == 32) return (r >> 2) & 3;
  else return (r ^ (r >> 3)) & 7;
}

// Maps workgroup L of the tiles of one kind (tm M-blocks x tn N-blocks) to
// (mb, nb): XCD L % 8 takes a contiguous range of tiles, N-block-major within
// the range, so the tiles running together on one XCD share a few weight
// blocks (resident in its L2) across many token blocks.
__device__ __forceinline__ void xcd_tile(int L, int tm, int tn, int& mb, int& nb, int gm) {
  const int count = tm * tn;
  if (count % 8 != 0 || tm % 8 != 0) { mb = L / tn; nb = L % tn; return; }
  const int per = tm >> 3;                           // M-blocks per XCD
  const int x = L & 7, j = L >> 3;                   // XCD, index within its range
  if (gm <= 0 || per % gm != 0) { nb = j / per; mb = x * per + j % per; return; }
  // groups of gm M-blocks: within a group the N-blocks advance slowest, so
  // the gm token blocks stay in L2 across the whole weight sweep
  const int grp = j / (gm * tn), r = j - grp * gm * tn;
  nb = r / gm;
  mb = x * per + grp * gm + r % gm;
}

// GELU of the exact erf form (nn.GELU(), approximate='none'), on the
// pre-activation rounded to bf16 first, as the reference's bf16 Linear
// hands it to GELU
__device__ __forceinline__ float gelu_of_bf16(float v) {
  const float r = (float)(bf16)v;
  return 0.5f * r * (1.f + erff(r * 0.70710678118654752f));
}

}  // namespace

// Argument block of each mode (MODE 0: the layer's projections; 1 and 2: the
// interaction generator's edge MLP, with the extra fields of EdgeGemmArgs).
// Outside the anonymous namespace: a kernel whose signature names an
// internal type gets internal linkage, and the compiler then treats its
// arguments differently (the MODE 0 kernel would no longer compile to the
// instructions of the projection GEMM as validated).
template <int MODE> struct GemmArgsOf { typedef EdgeGemmArgs type; };
template <> struct GemmArgsOf<0> { typedef QkvgArgs type; };

// FT features x TT tokens per workgroup, WF x WT waves (each FT/WF x TT/WT),
// NST pipeline stages of BK.
template <int FT, int TT, int WF, int WT, int BK, int NST> struct GemmCfg {
  static constexpr int kThreadsG = 64 * WF * WT;
  static constexpr int kCPR = BK / 8;                           // 16-byte chunks per tile row
  static constexpr int kWBytes = FT * BK * 2, kXBytes = TT * BK * 2;
  static constexpr int kStageBytes = kWBytes + kXBytes;
  static constexpr int kLds = NST * kStageBytes;
  static constexpr int kWLoads = kWBytes / 16 / kThreadsG, kXLoads = kXBytes / 16 / kThreadsG;
  static constexpr int kLoads = kWLoads + kXLoads;
  static constexpr int MI = FT / WF / 32, NJ = TT / WT / 32;   // MFMA tiles per wave
  static_assert(kWLoads * 16 * kThreadsG == kWBytes && kXLoads * 16 * kThreadsG == kXBytes, "tile split");
  static_assert(kLds <= 160 * 1024, "LDS");
  // the epilogue stages the tile in the ring's LDS: bf16 q/k/v tiles whole,
  // fp32 generator tiles in two halves of the tokens
  static_assert(TT * FT * 2 <= kLds && (TT / 2) * FT * 4 <= kLds, "epilogue staging exceeds the ring");
};

// MODE 0: q/k/v tiles and the additive generator's tiles (two K segments over
//         the token rows t and t+1, fp32 output): holo_qkvg_proj_fwd.
// MODE 1: q/k/v tiles and the edge MLP's hidden tiles (two K segments of W1,
//         weight row stride ldw, bias + exact GELU, bf16 output to hid):
//         holo_edge_hidden_fwd.
// MODE 2: one GEMM with an fp32 output, every tile a generator tile with one
//         K segment (the edge MLP's second layer): holo_gemm_f32out_fwd.
template <int FT, int TT, int WF, int WT, int BK, int NST, int WPE, int MODE>
__global__ void __launch_bounds__(64 * WF * WT) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_qkvg(typename GemmArgsOf<MODE>::type a) {
  using C = GemmCfg<FT, TT, WF, WT, BK, NST>;
  constexpr int NT = C::kThreadsG;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = w / WT, wt = w % WT;       // wave: feature slice, token slice

  // ---- tile of this workgroup: generator tiles first (twice the K) ----
  const int L = blockIdx.x;
  const int n_gen_tiles = a.tm * a.tng;
  const bool gen = L < n_gen_tiles;
  int mb, nb;
  if (gen) xcd_tile(L, a.tm, a.tng, mb, nb, a.group_m);
  else xcd_tile(L - n_gen_tiles, a.tm, a.tnq, mb, nb, a.group_m);
  const int64_t m0 = (int64_t)mb * TT;
  const int n0 = nb * FT;
  const int nseg = gen ? (MODE == 2 ? 1 : 2) : 1;
  const int nks = a.K / BK;                   // K steps per segment
  const int nit = nseg * nks;

  // ---- buffer resources: out-of-range rows read as zero ----
  const int n_rows_w = gen ? a.n_gen : a.n_qkv;
  // MODE 1: a weight of n rows with row stride ldw (>= K) is read as the range
  // from its first element to the last element of its last row, so the
  // second K segment (W1 + K) never reaches past W1's end
  int wbytes;
  if constexpr (MODE == 1) wbytes = (int)(((int64_t)(n_rows_w - 1) * (gen ? a.ldw : (int64_t)a.K) + a.K) * 2);
  else wbytes = (int)((int64_t)n_rows_w * a.K * 2);
  const __amdgpu_buffer_rsrc_t wr0 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(gen ? a.wg0 : a.wq), 0, wbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t wr1 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(gen ? a.wg1 : a.wq), 0, wbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(a.x), 0, (int)(a.M * a.ldx * 2), kBufferWord3);

  // ---- per-lane byte offsets of this thread's loads: chunk p = i*NT + tid
  // of a tile lands at LDS chunk p, so the lane fetches (row, logical chunk)
  // = (p / CPR, (p % CPR) ^ f(row)) ----
  int wo[C::kWLoads], xo0[C::kXLoads], xo1[C::kXLoads];
  static_for<C::kWLoads>([&](auto i) {
    const int p = i * NT + tid, r = p / C::kCPR, c = (p % C::kCPR) ^ gemm_swz<BK>(r);
    if constexpr (MODE == 1) wo[i] = (int)(((n0 + r) * (gen ? a.ldw : (int64_t)a.K) + c * 8) * 2);
    else wo[i] = ((n0 + r) * a.K + c * 8) * 2;
  });
  static_for<C::kXLoads>([&](auto i) {
    const int p = i * NT + tid, r = p / C::kCPR, c = (p % C::kCPR) ^ gemm_swz<BK>(r);
    const int64_t m = m0 + r;
    xo0[i] = (int)((m * a.ldx + c * 8) * 2);
    // shifted rows: token t+1 of the same sequence (t = T-1 wraps to 0); rows
    // past M stay past M (read as zero)
    const int64_t ms = m >= a.M ? m : ((m + 1) % a.T == 0 ? m + 1 - a.T : m + 1);
    xo1[i] = (int)((ms * a.ldx + c * 8) * 2);
  });

  auto issue = [&](int it, auto st) {
    const int seg = it >= nks, k0 = (it - seg * nks) * BK;
    unsigned char* ws = smem + decltype(st)::value * C::kStageBytes;
    unsigned char* xs = ws + C::kWBytes;
    static_for<C::kWLoads>([&](auto i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(seg ? wr1 : wr0, (lds_void*)(ws + (i * NT + 64 * w) * 16), 16,
                                               wo[i], k0 * 2, 0, 0);
    });
    static_for<C::kXLoads>([&](auto i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(xs + (i * NT + 64 * w) * 16), 16,
                                               seg ? xo1[i] : xo0[i], k0 * 2, 0, 0);
    });
  };

  // fragment reads: row lr of a 32-row block, logical chunk 2s+g. With
  // BK = 32 f(row) does not depend on the block; with BK = 64 it alternates
  // between even and odd 32-row blocks (row bit 5 enters through r >> 3), so
  // per substep one offset per block parity
  constexpr int RB = BK * 2;                  // bytes per tile row
  constexpr int NS = BK / 16;                 // k16 substeps per step
  int ko[2][NS];
  static_for<NS>([&](auto s) {
    ko[0][s] = lr * RB + ((2 * s + g) ^ gemm_swz<BK>(lr)) * 16;
    ko[1][s] = lr * RB + ((2 * s + g) ^ gemm_swz<BK>(lr + 32)) * 16;
  });
  const int wbase = wf * (FT / WF) * RB, xbase = C::kWBytes + wt * (TT / WT) * RB;

  f32x16 acc[C::MI][C::NJ];
  static_for<C::MI>([&](auto i) { static_for<C::NJ>([&](auto j) { acc[i][j] = f32x16{}; }); });

  auto compute = [&](auto st) {
    const unsigned char* sb = smem + decltype(st)::value * C::kStageBytes;
    static_for<NS>([&](auto s) {
      bf16x8 af[C::MI], bfr[C::NJ];
      // the wave's first block of each operand is 32-row aligned at an even
      // block index (FT/WF and TT/WT are multiples of 64)
      static_for<C::MI>([&](auto i) {
        af[i] = *reinterpret_cast<const bf16x8*>(sb + wbase + ko[i & 1][s] + i * 32 * RB);
      });
      static_for<C::NJ>([&](auto j) {
        bfr[j] = *reinterpret_cast<const bf16x8*>(sb + xbase + ko[j & 1][s] + j * 32 * RB);
      });
      static_for<C::MI>([&](auto i) {
        static_for<C::NJ>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        });
      });
    });
  };

  // one pipeline step: tile `it` in stage ST; up to NST-2 later tiles in flight
  auto step = [&](int it, auto st) {
    if (it >= nit) return;
    const int ahead = nit - 1 - it < NST - 2 ? nit - 1 - it : NST - 2;   // later tiles already issued
    if constexpr (NST >= 4) {
      if (ahead >= 2) wait_vmem<2 * C::kLoads>();
      else if (ahead == 1) wait_vmem<C::kLoads>();
      else wait_vmem<0>();
    } else {
      if (ahead >= 1) wait_vmem<C::kLoads>();
      else wait_vmem<0>();
    }
    ring_barrier();
    using SN = std::integral_constant<int, (decltype(st)::value + NST - 1) % NST>;
    if (it + NST - 1 < nit) issue(it + NST - 1, SN{});
    compute(st);
  };

  static_for<NST - 1>([&](auto i) { if (i < nit) issue(i, i); });
  for (int it = 0; it < nit; it += NST) {
    static_for<NST>([&](auto i) { step(it + i, i); });
  }

  // ---- epilogue: the tile goes through LDS (both stages are free once every
  // wave is past its last compute) so that global stores are whole 16-byte
  // pieces of token rows: lane = token, register quad q = 4 consecutive
  // features. Staged rows: token-major, the 16-byte chunk c of row r at
  // c ^ (r & xm), xm = min(cpr, 32) - 1 (the XOR stays inside the row;
  // conflict-free for the 32 token rows a store covers and for the row-wise
  // reads). The fp32 generator tile goes in two halves of the tokens (128 KB
  // each). ----
  ring_barrier();
  // generator tiles leave in fp32 (MODE 0, 2) or, MODE 1's hidden tiles, in bf16
  const bool f32out = gen && MODE != 1;
  const int es = f32out ? 4 : 2;                      // output bytes per element
  const int rowb = FT * es;                           // staged row bytes (512 or 1024)
  const int cpr = rowb / 16;                          // 16-byte chunks per staged row
  const int xm = (cpr < 32 ? cpr : 32) - 1;           // XOR mask: stays inside the row
  const int passes = f32out ? 2 : 1;
  const int tp = TT / passes;                         // tokens per pass
  const int n_out = gen ? a.n_gen : a.n_qkv;
  for (int hp = 0; hp < passes; ++hp) {
    const int tw0 = wt * (TT / WT);                   // first token of this wave
    if (tw0 / tp == hp) {
      static_for<C::NJ>([&](auto j) {
        const int r = tw0 % tp + j * 32 + lr;         // staged row (token)
        static_for<C::MI>([&](auto i) {
          static_for<4>([&](auto q) {
            const int f = wf * (FT / WF) + i * 32 + 8 * q + 4 * g;   // first of 4 features
            const f32x16& c = acc[i][j];
            // (the condition names `gen`, not f32out: capturing another
            // variable here changes how the compiler schedules MODE 0)
            if (MODE != 1 && gen) {
              const int ch = (f >> 2) ^ (r & xm);
              *reinterpret_cast<f32x4*>(smem + r * rowb + ch * 16) =
                  f32x4{c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]};
            } else {
              const int ch = (f >> 3) ^ (r & xm);
              if constexpr (MODE == 1) {
                if (gen) {                            // hidden tile: GELU(sum + bias) in bf16
                  // buffer load of the 4 biases: features past n_gen read as zero
                  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
                      const_cast<bf16*>(a.bias), 0, a.n_gen * 2, kBufferWord3);
                  const u32x2 raw = __builtin_amdgcn_raw_buffer_load_b64(br, (n0 + f) * 2, 0, 0);
                  const bf16x4 bv = __builtin_bit_cast(bf16x4, raw);
                  *reinterpret_cast<bf16x4*>(smem + r * rowb + ch * 16 + (f & 4) * 2) =
                      bf16x4{(bf16)gelu_of_bf16(c[4 * q] + (float)bv[0]), (bf16)gelu_of_bf16(c[4 * q + 1] + (float)bv[1]),
                             (bf16)gelu_of_bf16(c[4 * q + 2] + (float)bv[2]), (bf16)gelu_of_bf16(c[4 * q + 3] + (float)bv[3])};
                  return;
                }
              }
              *reinterpret_cast<bf16x4*>(smem + r * rowb + ch * 16 + (f & 4) * 2) =
                  bf16x4{(bf16)c[4 * q], (bf16)c[4 * q + 1], (bf16)c[4 * q + 2], (bf16)c[4 * q + 3]};
            }
          });
        });
      });
    }
    ring_barrier();
    for (int idx = tid; idx < tp * cpr; idx += NT) {
      const int r = idx / cpr, c = idx - r * cpr;
      const int64_t m = m0 + hp * tp + r;
      const int n = n0 + c * 16 / es;
      if (m >= a.M || n >= n_out) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + r * rowb + (c ^ (r & xm)) * 16);
      char* dst;
      if constexpr (MODE == 1) dst = gen ? reinterpret_cast<char*>(a.hid + m * a.ldh + n) : reinterpret_cast<char*>(a.qkv + m * a.ldq + n);
      else dst = gen ? reinterpret_cast<char*>(a.g + m * a.ldg + n) : reinterpret_cast<char*>(a.qkv + m * a.ldq + n);
      // non-temporal: the outputs (503 MB at config 2) stream to HBM instead
      // of evicting the token rows the other tiles still read (3% measured)
      if (n + 16 / es <= n_out) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
      else __builtin_nontemporal_store(v.xy, reinterpret_cast<u32x2*>(dst));   // bf16 tail of 4 features
    }
    if (hp + 1 < passes) ring_barrier();
  }
}

template <int FT, int TT, int WF, int WT, int BK, int NST, int WPE, int MODE>
static hipError_t launch_cfg(typename GemmArgsOf<MODE>::type a, hipStream_t s) {
  using C = GemmCfg<FT, TT, WF, WT, BK, NST>;
  a.tm = (int)((a.M + TT - 1) / TT);
  a.tnq = (a.n_qkv + FT - 1) / FT;
  a.tng = (a.n_gen + FT - 1) / FT;
  const hipError_t attr = allow_dynamic_lds<&gemm_qkvg<FT, TT, WF, WT, BK, NST, WPE, MODE>>();
  if (attr != hipSuccess) return attr;
  const unsigned grid = (unsigned)(a.tm * (a.tng + a.tnq));
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_qkvg<FT, TT, WF, WT, BK, NST, WPE, MODE>), dim3(grid), dim3(C::kThreadsG), C::kLds, s, a);
  return hipGetLastError();
}

// 256 features x 256 tokens per workgroup, 8 waves of 64 features x 128
// tokens (two per SIMD), K steps of 64 through two LDS stages (128 KB), token
// blocks grouped by 8 per weight sweep within each XCD. (Waves of 128 x 64:
// 1-2% slower.)
hipError_t launch_qkvg(const QkvgArgs& a, hipStream_t s) {
  QkvgArgs b = a;
  b.group_m = 8;
  return launch_cfg<256, 256, 4, 2, 64, 2, 2, 0>(b, s);
}

// the edge MLP on the same tiling (hidden layer with q/k/v tiles; second layer)
hipError_t launch_edge_hidden(const EdgeGemmArgs& a, hipStream_t s) {
  EdgeGemmArgs b = a;
  b.group_m = 8;
  return launch_cfg<256, 256, 4, 2, 64, 2, 2, 1>(b, s);
}

hipError_t launch_gemm_f32out(const EdgeGemmArgs& a, hipStream_t s) {
  EdgeGemmArgs b = a;
  b.group_m = 8;
  b.n_qkv = 0;
  b.wg1 = b.wg0;                 // one K segment: the second resource is never read
  return launch_cfg<256, 256, 4, 2, 64, 2, 2, 2>(b, s);
}

}  // namespace holo
