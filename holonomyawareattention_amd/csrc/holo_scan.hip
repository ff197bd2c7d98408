// Link rotations, chunked prefix-product scan and key/value transport (gfx950).
//
// Reference behaviour (core/attention_fast_chunked.py):
//   a_t   = edge_scale * (gq_t + gk_{(t+1) mod T})        additive   :80-84
//   (gq/gk are read in their own dtype GT, normally fp32, and composed in fp32)
//   a_t   = edge_scale * g_t                               direct a   :73-79
//   G_t   = exp(skew(a_t))                                 :86-87, core/utils.py:4-52
//   P_0 = I, P_{t+1} = G_t P_t ; Hol = G_{T-1} P_{T-1}     :89-95
//   qh_t  = P_t^T q_t, kh_t = P_t^T k_t, vh_t = P_t^T v_t   :108-110
//
// q, k, v are read in their storage type IO; the transported qh, kh, vh are
// written in the operand type OP of the attention that consumes them (fp32,
// bf16, or fp16 on the bf16 inference path: 11-bit significands for the
// matrix-core operands). A value beyond OP's finite range sets bit 1 of the
// status word in the workspace (bit 0: carry-wait time-out).
// Each 3x3 block of every (b, h) is an independent scan over t. The scan is
// one pass over the inputs in chunks of 64 links, one workgroup per
// (b, h, chunk):
//   1. link quaternions of the chunk's links -> LDS;
//   2. prefixes within the chunk over all threads (8 segments of 8 links per
//      block) and the chunk product T_c, published at once; the product of
//      all earlier chunks C_c = incl[c-1], read from the previous chunk when
//      it has published it, otherwise composed as T_{c-1} ... T_{c0}
//      incl[c0-1] from the products of the earlier chunks of its group of 8
//      (c0 = 16 floor(c/16)) and the group boundary's prefix, so a lagging
//      chain advances one group per hop instead of one chunk; then
//      incl[c] = T_c C_c is published (a chained scan through the workspace);
//   3. all threads: P_t, written to P, and the transported qh, kh, vh.
// Workgroups take chunks in ticket order (a global counter), chunk-major, so a
// chunk only ever waits on chunks that were handed out earlier and are running
// or done: the waits always end. Polls are bounded anyway; a time-out
// (impossible in a conforming launch) sets a flag in the workspace and the
// chunk's outputs become NaN. C_c is always the same nested product
// T_{c-1} (T_{c-2} (... (T_0 I))), so the composition order, and every bit of
// the result, does not depend on timing.
// Threads of a wave cover consecutive blocks of the same token rows, so the
// token-major input rows are read contiguously.
#include "holo_chain.h"
#include "holo_kernels.h"

namespace holo {

// link parameters of edge t (0 <= t < T) for head h, block blk
template <typename GT>
__device__ inline quat link_quat(const ScanArgs& a, int b, int h, int blk, int64_t t) {
  const GT* gq = reinterpret_cast<const GT*>(a.gq) + (b * a.T + t) * a.gq_rs + h * a.gq_hs + 3 * blk;
  float p0 = to_f32(gq[0]), p1 = to_f32(gq[1]), p2 = to_f32(gq[2]);
  if (a.gen_mode == 0) {
    int64_t tn = (t + 1 == a.T) ? 0 : t + 1;
    const GT* gk = reinterpret_cast<const GT*>(a.gk) + (b * a.T + tn) * a.gk_rs + h * a.gk_hs + 3 * blk;
    p0 += to_f32(gk[0]); p1 += to_f32(gk[1]); p2 += to_f32(gk[2]);
  }
  return qexp_skew(p0 * a.edge_scale, p1 * a.edge_scale, p2 * a.edge_scale);
}

size_t scan_state_bytes(int B, int64_t T, int H, int d) {
  const int64_t nch = padded_seq(T) / kChunk;
  return (size_t)B * H * 2 * nch * (d / 3) * 4 * sizeof(float) + 256;
}

// clears the chained-scan state and the ticket counter before every scan
// (atomic stores, so no cached copy of the old state survives)
__global__ void __launch_bounds__(256) scan_reset(uint64_t* state, int64_t n_pairs, unsigned* ticket) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n_pairs) __hip_atomic_store(state + i, ~(uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (i == 0) {
    __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ticket + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// (b*H + h, chunk) of this workgroup from the ticket counter, chunk-major
__device__ __forceinline__ void take_ticket(const ScanArgs& a, int64_t& bh, int64_t& c) {
  __shared__ unsigned s_ticket;
  if (threadIdx.x == 0)
    s_ticket = __hip_atomic_fetch_add(a.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int64_t tk = s_ticket, nbh = (int64_t)a.B * a.H;
  c = tk / nbh;             // >= nch only if the counter was not reset (caller returns)
  bh = tk % nbh;
}

// A published slot of the chained state (a chunk product, or a group's
// prefix), waited for with bounded polls. Waiting for exactly these values
// (rather than composing whatever predecessor state happens to be ready)
// keeps the association, and so every bit of the result, independent of
// timing.
__device__ inline quat wait_slot(const ScanArgs& a, const float* slot) {
  quat x;
  for (int polls = 0; polls < kMaxPolls; ++polls) {
    if (get_quat(slot, x)) return x;
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_fetch_or(a.ticket + 1, kStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float nan = __uint_as_float(kCanonNan);
  return quat{nan, nan, nan, nan};
}

// Steps 2-3 of the scan, all threads of the workgroup (thread tid < 8*nb
// owns segment seg = tid / nb, links 8seg .. 8seg+7, of block blk = tid % nb).
// On entry gs slot (r, blk) holds the link quaternion of link t0 + r
// (identity past T-2); on return it holds P_{t0+r}, P is written for
// t0 + r < T, the chunk's inclusive prefix is published and, from the last
// chunk, the holonomy is written. Association (fixed, so results do not
// depend on timing): segment-local prefixes, then the product E of the
// earlier segments, then P = (segment prefix) (E C) with C the product of all
// earlier chunks. ss: 8*nb quaternions of LDS, cs: nb.
template <typename GT>
__device__ inline void chunk_prefix(const ScanArgs& a, float* gs, float* ss, float* cs, int64_t bh, int64_t c,
                                    int tid) {
  const int nb = a.nb;
  const int seg = tid / (nb > 0 ? nb : 1), blk = tid - seg * nb;
  const bool act = tid < 8 * nb;
  if (act) {
    quat p = qident();
    for (int r = 8 * seg; r < 8 * seg + 8; ++r) {       // segment-local exclusive prefixes
      float* slot = &gs[(r * nb + blk) * 4];
      const quat g = load_quat(slot);
      store_quat(slot, p);
      p = qmul(g, p);
    }
    store_quat(&ss[(seg * nb + blk) * 4], p);           // segment product
  }
  __syncthreads();
  quat E = qident();                                    // product of the earlier segments
  if (act) {
    for (int k = 0; k < seg; ++k) E = qmul(load_quat(&ss[(k * nb + blk) * 4]), E);
    if (seg == 7) {
      const quat Tc = qmul(load_quat(&ss[(7 * nb + blk) * 4]), E);       // chunk product
      // C_c = T_{c-1} (T_{c-2} (... (T_{c0} incl[c0-1]))) = incl[c-1]: taken
      // from incl[c-1] when chunk c-1 has published it, otherwise composed
      // from the group boundary's incl[c0-1] and the products T_j of the
      // group's earlier chunks (published before any wait). Both give the
      // same bits (same nesting, context-independent qmul), so the result
      // does not depend on which one was ready.
      const int64_t c0 = c / kScanGroup * kScanGroup;
      float* tot = a.incl + (bh * a.nch * nb + blk) * 4;                 // T_j at tot[j * nb * 4]
      float* inc = a.incl + ((int64_t)a.B * a.H * a.nch + bh * a.nch) * nb * 4 + blk * 4;   // incl[j]
      if (c - c0 < kScanGroup - 1 && c + 1 < a.nch) put_quat(tot + c * nb * 4, Tc);   // read by the group's later chunks
      quat C = qident();
      if (c > 0 && !get_quat(inc + (c - 1) * nb * 4, C)) {
        if (c == c0) {
          C = wait_slot(a, inc + (c - 1) * nb * 4);
        } else {
          C = c0 == 0 ? qident() : wait_slot(a, inc + (c0 - 1) * nb * 4);
          for (int64_t j = c0; j < c; j += 4) {      // four products per memory round trip
            quat tj[4];
            bool ok[4];
            static_for<4>([&](auto i) { ok[i] = j + i < c ? get_quat(tot + (j + i) * nb * 4, tj[i]) : true; });
            static_for<4>([&](auto i) {
              if (j + i < c) {
                if (!ok[i]) tj[i] = wait_slot(a, tot + (j + i) * nb * 4);
                C = qmul(tj[i], C);
              }
            });
          }
        }
      }
      if (c + 1 < a.nch) put_quat(inc + c * nb * 4, qmul(Tc, C));
      store_quat(&cs[blk * 4], C);
    }
  }
  __syncthreads();
  if (act) {
    const quat X = qmul(E, load_quat(&cs[blk * 4]));
    const int64_t t0 = c * kChunk;
    const int64_t q0 = (bh * a.T + t0) * nb + blk;      // quaternion index of (t0, blk)
    for (int r = 8 * seg; r < 8 * seg + 8; ++r) {       // lanes of a wave: whole rows of P
      float* slot = &gs[(r * nb + blk) * 4];
      const quat p = qmul(load_quat(slot), X);
      store_quat(slot, p);
      if (t0 + r < a.T) {
        if (a.p_format) store_quat_snorm16_nt(reinterpret_cast<short*>(a.P) + (q0 + (int64_t)r * nb) * 4, p);
        else store_quat(a.P + (q0 + (int64_t)r * nb) * 4, p);
      }
    }
  }
  __syncthreads();
  if (a.hol && c == a.nch - 1 && tid < nb) {            // Hol = G_close P_{T-1}
    const int b = (int)(bh / a.H), h = (int)(bh % a.H);
    const int64_t n = a.T - c * kChunk;
    const quat pl = load_quat(&gs[((n - 1) * nb + tid) * 4]);
    store_quat(a.hol + (bh * nb + tid) * 4, qmul(link_quat<GT>(a, b, h, tid, a.T - 1), pl));
  }
}

// One workgroup per (b, h, chunk) tile of 64 tokens (any d <= 96):
//   1. all threads: link quaternions g_t of the tile's links -> LDS;
//   2-3. all threads: prefixes, the chained carry and P_t (chunk_prefix) ->
//      global P and LDS; qh = P^T q, kh = P^T k
//      and vh = P^T v into row-major qh, kh tiles and a transposed vh tile in
//      LDS (zero padding);
//   4. the tiles leave with 16-byte stores of whole rows (each tile is one
//      contiguous block in global memory).
// Sets the overflow bit of the status word when |x| exceeds OP's finite range
// for any value x this thread converts (mx: the largest magnitude seen).
template <typename OP>
__device__ __forceinline__ void note_range(const ScanArgs& a, float mx) {
  if constexpr (sizeof(OP) == 2 && !std::is_same<OP, bf16>::value) {
    if (mx > max_finite<OP>())
      __hip_atomic_fetch_or(a.ticket + 1, kStatusOverflow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <typename IO, typename OP, typename GT, int DP>
__global__ void __launch_bounds__(256) chunk_apply(ScanArgs a) {
  constexpr int E = 16 / sizeof(OP);
  constexpr int KS = DP + E;            // LDS row strides (16 B multiples)
  constexpr int VS = kChunk + E;
  constexpr int NBM = DP / 3;           // blocks held in LDS (nb <= NBM)
  constexpr int NBX = (DP + 2) / 3;     // 3-dim groups covering DP
  __shared__ __align__(16) float gs[kChunk * NBM * 4];
  __shared__ __align__(16) float ss[8 * NBM * 4];
  __shared__ __align__(16) float cs[NBM * 4];
  __shared__ __align__(16) OP qhs[kChunk * KS];
  __shared__ __align__(16) OP khs[kChunk * KS];
  __shared__ __align__(16) OP vts[DP * VS];

  const int tid = threadIdx.x;
  int64_t bh, c;
  take_ticket(a, bh, c);
  if (c >= a.nch) return;                 // uniform: every thread holds the same ticket
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int nb = a.nb;
  const int64_t t0 = c * kChunk;

  for (int idx = tid; idx < kChunk * nb; idx += 256) {
    int i = idx / nb, blk = idx % nb;
    int64_t t = t0 + i;
    quat g = (t + 1 < a.T) ? link_quat<GT>(a, b, h, blk, t) : qident();
    *reinterpret_cast<f32x4*>(&gs[idx * 4]) = f32x4{g.w, g.x, g.y, g.z};
  }
  __syncthreads();
  chunk_prefix<GT>(a, gs, ss, cs, bh, c, tid);
  const IO* qin = reinterpret_cast<const IO*>(a.q) + h * a.q_hs;
  const IO* kin = reinterpret_cast<const IO*>(a.k) + h * a.k_hs;
  const IO* vin = reinterpret_cast<const IO*>(a.v) + h * a.v_hs;
  float mx = 0.f;
  for (int idx = tid; idx < kChunk * NBX; idx += 256) {
    int i = idx / NBX, blk = idx % NBX, c0 = 3 * blk;
    int64_t t = t0 + i;
    float q3[3] = {0.f, 0.f, 0.f}, k3[3] = {0.f, 0.f, 0.f}, v3[3] = {0.f, 0.f, 0.f};
    if (t < a.T) {
      const IO* qr = qin + (b * a.T + t) * a.q_rs + c0;
      const IO* kr = kin + (b * a.T + t) * a.k_rs + c0;
      const IO* vr = vin + (b * a.T + t) * a.v_rs + c0;
      for (int j = 0; j < 3; ++j)
        if (c0 + j < a.d) { q3[j] = to_f32(qr[j]); k3[j] = to_f32(kr[j]); v3[j] = to_f32(vr[j]); }
      if (blk < nb) {
        const quat pt = load_quat(&gs[(i * nb + blk) * 4]);
        rot3 R = qmat(a.inert ? qconj(pt) : pt);          // R^T applied below: P^T u, or P u
        float y0, y1, y2;
        rot_t_apply(R, q3[0], q3[1], q3[2], y0, y1, y2);
        q3[0] = y0; q3[1] = y1; q3[2] = y2;
        rot_t_apply(R, k3[0], k3[1], k3[2], y0, y1, y2);
        k3[0] = y0; k3[1] = y1; k3[2] = y2;
        rot_t_apply(R, v3[0], v3[1], v3[2], y0, y1, y2);
        v3[0] = y0; v3[1] = y1; v3[2] = y2;
      }
    }
    for (int j = 0; j < 3; ++j) {
      mx = fmaxf(mx, fmaxf(fabsf(q3[j]), fmaxf(fabsf(k3[j]), fabsf(v3[j]))));
      if (c0 + j < DP) {
        qhs[i * KS + c0 + j] = from_f32<OP>(q3[j]);
        khs[i * KS + c0 + j] = from_f32<OP>(k3[j]);
        vts[(c0 + j) * VS + i] = from_f32<OP>(v3[j]);
      }
    }
  }
  note_range<OP>(a, mx);
  __syncthreads();
  u32x4* qdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.qh) + (bh * a.Tp + t0) * DP);
  u32x4* kdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.kh) + (bh * a.Tp + t0) * DP);
  u32x4* vdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.vh_t) + (bh * a.nch + c) * DP * kChunk);
  constexpr int KR = DP / E, VR = kChunk / E;      // 16 B chunks per row
  for (int i = tid; i < kChunk * KR; i += 256) {
    qdst[i] = *reinterpret_cast<const u32x4*>(&qhs[(i / KR) * KS + (i % KR) * E]);
    kdst[i] = *reinterpret_cast<const u32x4*>(&khs[(i / KR) * KS + (i % KR) * E]);
  }
  for (int i = tid; i < DP * VR; i += 256)
    vdst[i] = *reinterpret_cast<const u32x4*>(&vts[(i / VR) * VS + (i % VR) * E]);
}

// Wide path for d % 24 == 0 with 16-byte aligned rows: thread (i, g) owns token
// t0 + i and dims [24g, 24g + 24) (8 blocks) of one head. All of its global
// loads (link parameters of link t, query, key and value rows) are issued
// before any arithmetic, the query and key rows leave with 16-byte stores, and
// the value tile is transposed through LDS. NG = d / 24 threads per token.
template <int N> struct VecOf { typedef unsigned int type __attribute__((ext_vector_type(N))); };

template <typename T, int N>   // N elements of T starting at a 16-byte aligned p
__device__ __forceinline__ void load_row(const T* p, float* out) {
  constexpr int E = 16 / sizeof(T);
  static_for<N / E>([&](auto c) {
    u32x4 raw = reinterpret_cast<const u32x4*>(p)[c];
    const T* e = reinterpret_cast<const T*>(&raw);
    static_for<E>([&](auto j) { out[c * E + j] = to_f32(e[j]); });
  });
}

template <typename T, int N>
__device__ __forceinline__ void store_row(T* p, const float* in) {
  constexpr int E = 16 / sizeof(T);
  static_for<N / E>([&](auto c) {
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
    static_for<E>([&](auto j) { e[j] = from_f32<T>(in[c * E + j]); });
    reinterpret_cast<u32x4*>(p)[c] = raw;
  });
}

template <typename IO, typename OP, typename GT, int NG, int DP, bool DIRECT>
__global__ void __launch_bounds__(64 * NG) chunk_apply_wide(ScanArgs a) {
  constexpr int NT = 64 * NG;           // threads
  constexpr int NB = 8 * NG;            // blocks per head (nb)
  constexpr int D = 24 * NG;            // head dimension
  constexpr int E = 16 / sizeof(OP);
  constexpr int VS = kChunk + E;
  constexpr int KS = DP + E;             // row stride of the staged qh / kh tiles
  constexpr int GS_BYTES = kChunk * NB * 16, QK_BYTES = 2 * kChunk * KS * (int)sizeof(OP);
  // link quaternions / P, later reused for the transported qh and kh tiles
  // (packing both phases and the value tile into 38 KB, four workgroups per
  // CU, measured 1.5% slower at d = 96)
  __shared__ __align__(16) float gs[(GS_BYTES > QK_BYTES ? GS_BYTES : QK_BYTES) / 4];
  __shared__ __align__(16) float ss[8 * NB * 4];
  __shared__ __align__(16) float cs[NB * 4];
  __shared__ __align__(16) OP vts[DP * VS];
  OP* const qts = reinterpret_cast<OP*>(gs);
  OP* const kts = qts + kChunk * KS;

  const int tid = threadIdx.x;
  const int i = tid / NG, g = tid % NG;
  int64_t bh, c;
  take_ticket(a, bh, c);
  if (c >= a.nch) return;                 // uniform: every thread holds the same ticket
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int64_t t0 = c * kChunk, t = t0 + i;

  // ---- all global loads first ----
  float gq[24], gk[24], qv[24], kv[24], vv[24];
  const bool link = t + 1 < a.T;
  if (link) {
    load_row<GT, 24>(reinterpret_cast<const GT*>(a.gq) + (b * a.T + t) * a.gq_rs + h * a.gq_hs + 24 * g, gq);
    if constexpr (!DIRECT) {
      load_row<GT, 24>(reinterpret_cast<const GT*>(a.gk) + (b * a.T + t + 1) * a.gk_rs + h * a.gk_hs + 24 * g, gk);
    }
  }
  if constexpr (DIRECT) static_for<24>([&](auto j) { gk[j] = 0.f; });
  const bool tok = t < a.T;
  if (tok) {
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.q) + (b * a.T + t) * a.q_rs + h * a.q_hs + 24 * g, qv);
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.k) + (b * a.T + t) * a.k_rs + h * a.k_hs + 24 * g, kv);
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.v) + (b * a.T + t) * a.v_rs + h * a.v_hs + 24 * g, vv);
  } else {
    static_for<24>([&](auto j) { qv[j] = 0.f; kv[j] = 0.f; vv[j] = 0.f; });
  }
  // ---- link quaternions of link t -> LDS ----
  static_for<8>([&](auto j) {
    quat q = qident();
    if (link) {
      const float es = a.edge_scale;
      q = qexp_skew((gq[3 * j] + gk[3 * j]) * es, (gq[3 * j + 1] + gk[3 * j + 1]) * es,
                    (gq[3 * j + 2] + gk[3 * j + 2]) * es);
    }
    *reinterpret_cast<f32x4*>(&gs[(i * NB + 8 * g + j) * 4]) = f32x4{q.w, q.x, q.y, q.z};
  });
  __syncthreads();
  // ---- prefixes: gs slots become P_t, P written, carry chained ----
  chunk_prefix<GT>(a, gs, ss, cs, bh, c, tid);
  // ---- transport: kh row to global, vh into the transposed tile ----
  static_for<8>([&](auto j) {
    const quat pt = load_quat(&gs[(i * NB + 8 * g + j) * 4]);
    rot3 R = qmat(a.inert ? qconj(pt) : pt);              // R^T applied below: P^T u, or P u
    float y0, y1, y2;
    rot_t_apply(R, qv[3 * j], qv[3 * j + 1], qv[3 * j + 2], y0, y1, y2);
    qv[3 * j] = y0; qv[3 * j + 1] = y1; qv[3 * j + 2] = y2;
    rot_t_apply(R, kv[3 * j], kv[3 * j + 1], kv[3 * j + 2], y0, y1, y2);
    kv[3 * j] = y0; kv[3 * j + 1] = y1; kv[3 * j + 2] = y2;
    rot_t_apply(R, vv[3 * j], vv[3 * j + 1], vv[3 * j + 2], y0, y1, y2);
    vv[3 * j] = y0; vv[3 * j + 1] = y1; vv[3 * j + 2] = y2;
  });
  if constexpr (sizeof(OP) == 2 && !std::is_same<OP, bf16>::value) {
    float mx = 0.f;
    static_for<24>([&](auto j) { mx = fmaxf(mx, fmaxf(fabsf(qv[j]), fmaxf(fabsf(kv[j]), fabsf(vv[j])))); });
    note_range<OP>(a, mx);
  }
  // ---- stage the three transported tiles in LDS (the P slots are free once
  // every thread has read its own), then write each with whole 16-byte rows
  // per lane: the qh and kh tiles of a chunk are contiguous 64 x DP blocks ----
  __syncthreads();
  // zero the padded rows of the value tile
  for (int idx = tid; idx < (DP - D) * kChunk; idx += NT)
    vts[(D + idx / kChunk) * VS + idx % kChunk] = from_f32<OP>(0.f);
  store_row<OP, 24>(qts + i * KS + 24 * g, qv);
  store_row<OP, 24>(kts + i * KS + 24 * g, kv);
  if (DP > D && g == NG - 1) {
    float z[DP > D ? DP - D : E];
    static_for<(DP > D ? DP - D : E)>([&](auto j) { z[j] = 0.f; });
    if constexpr (DP > D) {
      store_row<OP, DP - D>(qts + i * KS + D, z);
      store_row<OP, DP - D>(kts + i * KS + D, z);
    }
  }
  static_for<24>([&](auto j) { vts[(24 * g + j) * VS + i] = from_f32<OP>(vv[j]); });
  __syncthreads();
  u32x4* qdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.qh) + (bh * a.Tp + t0) * DP);
  u32x4* kdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.kh) + (bh * a.Tp + t0) * DP);
  constexpr int KR = DP / E;
  // non-temporal stores: the outputs stream to HBM (the attention reads them
  // back after the whole scan) instead of evicting the inputs in flight
  for (int idx = tid; idx < kChunk * KR; idx += NT) {
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&qts[(idx / KR) * KS + (idx % KR) * E]), qdst + idx);
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&kts[(idx / KR) * KS + (idx % KR) * E]), kdst + idx);
  }
  u32x4* vdst = reinterpret_cast<u32x4*>(reinterpret_cast<OP*>(a.vh_t) + (bh * a.nch + c) * DP * kChunk);
  constexpr int VR = kChunk / E;
  for (int idx = tid; idx < DP * VR; idx += NT)
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&vts[(idx / VR) * VS + (idx % VR) * E]), vdst + idx);
}

hipError_t launch_chain_reset(void* state, int64_t n_pairs, unsigned* ticket, hipStream_t s) {
  const int tpb = 256;
  hipLaunchKernelGGL(scan_reset, dim3((unsigned)((n_pairs + tpb - 1) / tpb > 0 ? (n_pairs + tpb - 1) / tpb : 1)),
                     dim3(tpb), 0, s, reinterpret_cast<uint64_t*>(state), n_pairs, ticket);
  return hipGetLastError();
}

template <typename IO, typename OP, typename GT>
hipError_t launch_scan(const ScanArgs& a, hipStream_t s) {
  const int tpb = 256;
  const int64_t n_pairs = (int64_t)a.B * a.H * 2 * a.nch * a.nb * 2;    // 64-bit words of the state
  hipLaunchKernelGGL(scan_reset, dim3((unsigned)((n_pairs + tpb - 1) / tpb > 0 ? (n_pairs + tpb - 1) / tpb : 1)),
                     dim3(tpb), 0, s, reinterpret_cast<uint64_t*>(a.incl), n_pairs, a.ticket);
  const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nch));
  if (a.wide) {
    const bool direct = a.gen_mode == 1;
    switch (a.d) {
      case 48:
        if (direct) hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 2, 64, true>), grid, dim3(128), 0, s, a);
        else hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 2, 64, false>), grid, dim3(128), 0, s, a);
        break;
      case 72:
        if (direct) hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 3, 96, true>), grid, dim3(192), 0, s, a);
        else hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 3, 96, false>), grid, dim3(192), 0, s, a);
        break;
      case 96:
        if (direct) hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 4, 96, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((chunk_apply_wide<IO, OP, GT, 4, 96, false>), grid, dim3(256), 0, s, a);
        break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (a.Dp) {
    case 32: hipLaunchKernelGGL((chunk_apply<IO, OP, GT, 32>), grid, dim3(tpb), 0, s, a); break;
    case 64: hipLaunchKernelGGL((chunk_apply<IO, OP, GT, 64>), grid, dim3(tpb), 0, s, a); break;
    case 96: hipLaunchKernelGGL((chunk_apply<IO, OP, GT, 96>), grid, dim3(tpb), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template hipError_t launch_scan<float, float, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, bf16, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, bf16, bf16>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, f16, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, f16, bf16>(const ScanArgs&, hipStream_t);

}  // namespace holo
