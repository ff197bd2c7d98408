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
// Each 3x3 block of every (b, h) is an independent scan over t. The scan runs
// in three launches over chunks of 64 links:
//   1. chunk_totals : one thread per (b, chunk, h, block) composes the chunk's
//                     64 link rotations (quaternions) into the chunk total;
//   2. chunk_carry  : one thread per (b, h, block) composes the totals in chunk
//                     order into exclusive carries (the prefix P at each chunk
//                     start) and the holonomy;
//   3. chunk_apply  : one workgroup per (b, chunk, h) starts each block from
//                     its carry, recomposes the chunk link by link, writes P_t
//                     and the transported kh, vh tiles (zero padding included).
// Threads of a wave cover consecutive blocks of the same token rows, so the
// token-major input rows are read contiguously.
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

template <typename GT>
__global__ void __launch_bounds__(256) chunk_totals(ScanArgs a) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t n = (int64_t)a.B * a.nch * a.H * a.nb;
  if (gid >= n) return;
  int blk = gid % a.nb;
  int h = (gid / a.nb) % a.H;
  int64_t c = (gid / ((int64_t)a.nb * a.H)) % a.nch;
  int b = gid / ((int64_t)a.nb * a.H * a.nch);
  int64_t t0 = c * kChunk;
  int64_t t1 = t0 + kChunk;
  if (t1 > a.T - 1) t1 = a.T - 1;      // links 0..T-2 only
  quat acc = qident();
  for (int64_t t = t0; t < t1; ++t) acc = qmul(link_quat<GT>(a, b, h, blk, t), acc);
  store_quat(a.totals + (((int64_t)b * a.H + h) * a.nch + c) * a.nb * 4 + blk * 4, acc);
}

template <typename GT>
__global__ void __launch_bounds__(256) chunk_carry(ScanArgs a) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t n = (int64_t)a.B * a.H * a.nb;
  if (gid >= n) return;
  int blk = gid % a.nb;
  int h = (gid / a.nb) % a.H;
  int b = gid / ((int64_t)a.nb * a.H);
  int64_t base = ((int64_t)b * a.H + h) * a.nch * a.nb * 4 + blk * 4;
  quat cur = qident();
  for (int64_t c = 0; c < a.nch; ++c) {
    int64_t off = base + c * a.nb * 4;
    store_quat(a.carry + off, cur);
    cur = qmul(load_quat(a.totals + off), cur);
  }
  if (a.hol) {   // cur == P_{T-1}
    quat g = link_quat<GT>(a, b, h, blk, a.T - 1);
    store_quat(a.hol + (((int64_t)b * a.H + h) * a.nb + blk) * 4, qmul(g, cur));
  }
}

// One workgroup per (b, chunk, h) tile of 64 tokens:
//   1. all threads: link quaternions g_t of the tile's links -> LDS;
//   2. one thread per block: P_t = g_{t-1} ... g_{t0} C (C = carry), written to
//      global P and over g_t in LDS;
//   3. all threads, one (token, 3-dim group) each: qh = P^T q, kh = P^T k and
//      vh = P^T v into row-major qh, kh tiles and a transposed vh tile in LDS
//      (zero padding);
//   4. the tiles leave with 16-byte stores of whole rows (each tile is one
//      contiguous block in global memory).
template <typename IO, typename GT, int DP>
__global__ void __launch_bounds__(256) chunk_apply(ScanArgs a) {
  constexpr int E = 16 / sizeof(IO);
  constexpr int KS = DP + E;            // LDS row strides (16 B multiples)
  constexpr int VS = kChunk + E;
  constexpr int NBM = DP / 3;           // blocks held in LDS (nb <= NBM)
  constexpr int NBX = (DP + 2) / 3;     // 3-dim groups covering DP
  __shared__ __align__(16) float gs[kChunk * NBM * 4];
  __shared__ __align__(16) IO qhs[kChunk * KS];
  __shared__ __align__(16) IO khs[kChunk * KS];
  __shared__ __align__(16) IO vts[DP * VS];

  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int64_t c = blockIdx.y;
  const int b = blockIdx.z;
  const int nb = a.nb;
  const int64_t t0 = c * kChunk;
  const int64_t bh = (int64_t)b * a.H + h;

  for (int idx = tid; idx < kChunk * nb; idx += 256) {
    int i = idx / nb, blk = idx % nb;
    int64_t t = t0 + i;
    quat g = (t + 1 < a.T) ? link_quat<GT>(a, b, h, blk, t) : qident();
    *reinterpret_cast<f32x4*>(&gs[idx * 4]) = f32x4{g.w, g.x, g.y, g.z};
  }
  __syncthreads();
  if (tid < nb) {
    quat p = load_quat(a.carry + (bh * a.nch + c) * nb * 4 + tid * 4);
    float* Pout = a.P + (bh * a.T + t0) * nb * 4 + tid * 4;
    for (int i = 0; i < kChunk; ++i) {
      float* slot = &gs[(i * nb + tid) * 4];
      quat g = load_quat(slot);
      store_quat(slot, p);
      if (t0 + i < a.T) store_quat(Pout + (int64_t)i * nb * 4, p);
      p = qmul(g, p);
    }
  }
  __syncthreads();
  const IO* qin = reinterpret_cast<const IO*>(a.q) + h * a.q_hs;
  const IO* kin = reinterpret_cast<const IO*>(a.k) + h * a.k_hs;
  const IO* vin = reinterpret_cast<const IO*>(a.v) + h * a.v_hs;
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
        rot3 R = qmat(load_quat(&gs[(i * nb + blk) * 4]));
        float y0, y1, y2;
        rot_t_apply(R, q3[0], q3[1], q3[2], y0, y1, y2);
        q3[0] = y0; q3[1] = y1; q3[2] = y2;
        rot_t_apply(R, k3[0], k3[1], k3[2], y0, y1, y2);
        k3[0] = y0; k3[1] = y1; k3[2] = y2;
        rot_t_apply(R, v3[0], v3[1], v3[2], y0, y1, y2);
        v3[0] = y0; v3[1] = y1; v3[2] = y2;
      }
    }
    for (int j = 0; j < 3; ++j)
      if (c0 + j < DP) {
        qhs[i * KS + c0 + j] = from_f32<IO>(q3[j]);
        khs[i * KS + c0 + j] = from_f32<IO>(k3[j]);
        vts[(c0 + j) * VS + i] = from_f32<IO>(v3[j]);
      }
  }
  __syncthreads();
  u32x4* qdst = reinterpret_cast<u32x4*>(reinterpret_cast<IO*>(a.qh) + (bh * a.Tp + t0) * DP);
  u32x4* kdst = reinterpret_cast<u32x4*>(reinterpret_cast<IO*>(a.kh) + (bh * a.Tp + t0) * DP);
  u32x4* vdst = reinterpret_cast<u32x4*>(reinterpret_cast<IO*>(a.vh_t) + (bh * a.nch + c) * DP * kChunk);
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

template <typename IO, typename GT, int NG, int DP>
__global__ void __launch_bounds__(64 * NG) chunk_apply_wide(ScanArgs a) {
  constexpr int NT = 64 * NG;           // threads
  constexpr int NB = 8 * NG;            // blocks per head (nb)
  constexpr int D = 24 * NG;            // head dimension
  constexpr int E = 16 / sizeof(IO);
  constexpr int VS = kChunk + E;
  __shared__ __align__(16) float gs[kChunk * NB * 4];
  __shared__ __align__(16) IO vts[DP * VS];

  const int tid = threadIdx.x;
  const int i = tid / NG, g = tid % NG;
  const int h = blockIdx.x;
  const int64_t c = blockIdx.y;
  const int b = blockIdx.z;
  const int64_t t0 = c * kChunk, t = t0 + i;
  const int64_t bh = (int64_t)b * a.H + h;

  // ---- all global loads first ----
  float gq[24], gk[24], qv[24], kv[24], vv[24];
  const bool link = t + 1 < a.T;
  if (link) {
    load_row<GT, 24>(reinterpret_cast<const GT*>(a.gq) + (b * a.T + t) * a.gq_rs + h * a.gq_hs + 24 * g, gq);
    if (a.gen_mode == 0) {
      load_row<GT, 24>(reinterpret_cast<const GT*>(a.gk) + (b * a.T + t + 1) * a.gk_rs + h * a.gk_hs + 24 * g, gk);
    } else {
      static_for<24>([&](auto j) { gk[j] = 0.f; });
    }
  }
  const bool tok = t < a.T;
  if (tok) {
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.q) + (b * a.T + t) * a.q_rs + h * a.q_hs + 24 * g, qv);
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.k) + (b * a.T + t) * a.k_rs + h * a.k_hs + 24 * g, kv);
    load_row<IO, 24>(reinterpret_cast<const IO*>(a.v) + (b * a.T + t) * a.v_rs + h * a.v_hs + 24 * g, vv);
  } else {
    static_for<24>([&](auto j) { qv[j] = 0.f; kv[j] = 0.f; vv[j] = 0.f; });
  }
  // zero the padded rows of the value tile
  for (int idx = tid; idx < (DP - D) * kChunk; idx += NT)
    vts[(D + idx / kChunk) * VS + idx % kChunk] = from_f32<IO>(0.f);

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
  // ---- chain: one thread per block, P_t from the chunk carry ----
  if (tid < NB) {
    quat p = load_quat(a.carry + (bh * a.nch + c) * NB * 4 + tid * 4);
    float* Pout = a.P + (bh * a.T + t0) * NB * 4 + tid * 4;
    int n = (int)(a.T - t0 < kChunk ? a.T - t0 : kChunk);
#pragma unroll 4
    for (int r = 0; r < n; ++r) {
      float* slot = &gs[(r * NB + tid) * 4];
      quat gl = load_quat(slot);
      store_quat(slot, p);
      store_quat(Pout + (int64_t)r * NB * 4, p);
      p = qmul(gl, p);
    }
  }
  __syncthreads();
  // ---- transport: kh row to global, vh into the transposed tile ----
  static_for<8>([&](auto j) {
    rot3 R = qmat(load_quat(&gs[(i * NB + 8 * g + j) * 4]));
    float y0, y1, y2;
    rot_t_apply(R, qv[3 * j], qv[3 * j + 1], qv[3 * j + 2], y0, y1, y2);
    qv[3 * j] = y0; qv[3 * j + 1] = y1; qv[3 * j + 2] = y2;
    rot_t_apply(R, kv[3 * j], kv[3 * j + 1], kv[3 * j + 2], y0, y1, y2);
    kv[3 * j] = y0; kv[3 * j + 1] = y1; kv[3 * j + 2] = y2;
    rot_t_apply(R, vv[3 * j], vv[3 * j + 1], vv[3 * j + 2], y0, y1, y2);
    vv[3 * j] = y0; vv[3 * j + 1] = y1; vv[3 * j + 2] = y2;
  });
  IO* qrow = reinterpret_cast<IO*>(a.qh) + (bh * a.Tp + t) * DP;
  IO* krow = reinterpret_cast<IO*>(a.kh) + (bh * a.Tp + t) * DP;
  store_row<IO, 24>(qrow + 24 * g, qv);
  store_row<IO, 24>(krow + 24 * g, kv);
  if (DP > D && g == NG - 1) {
    float z[DP > D ? DP - D : E];
    static_for<(DP > D ? DP - D : E)>([&](auto j) { z[j] = 0.f; });
    if constexpr (DP > D) {
      store_row<IO, DP - D>(qrow + D, z);
      store_row<IO, DP - D>(krow + D, z);
    }
  }
  static_for<24>([&](auto j) { vts[(24 * g + j) * VS + i] = from_f32<IO>(vv[j]); });
  __syncthreads();
  u32x4* vdst = reinterpret_cast<u32x4*>(reinterpret_cast<IO*>(a.vh_t) + (bh * a.nch + c) * DP * kChunk);
  constexpr int VR = kChunk / E;
  for (int idx = tid; idx < DP * VR; idx += NT)
    vdst[idx] = *reinterpret_cast<const u32x4*>(&vts[(idx / VR) * VS + (idx % VR) * E]);
}

template <typename IO, typename GT>
hipError_t launch_scan(const ScanArgs& a, hipStream_t s) {
  const int tpb = 256;
  int64_t n1 = (int64_t)a.B * a.nch * a.H * a.nb;
  int64_t n2 = (int64_t)a.B * a.H * a.nb;
  if (n1 > 0) hipLaunchKernelGGL(chunk_totals<GT>, dim3((n1 + tpb - 1) / tpb), dim3(tpb), 0, s, a);
  if (n2 > 0) hipLaunchKernelGGL(chunk_carry<GT>, dim3((n2 + tpb - 1) / tpb), dim3(tpb), 0, s, a);
  dim3 grid(a.H, (unsigned)a.nch, a.B);
  if (a.wide) {
    switch (a.d) {
      case 48: hipLaunchKernelGGL((chunk_apply_wide<IO, GT, 2, 64>), grid, dim3(128), 0, s, a); break;
      case 72: hipLaunchKernelGGL((chunk_apply_wide<IO, GT, 3, 96>), grid, dim3(192), 0, s, a); break;
      case 96: hipLaunchKernelGGL((chunk_apply_wide<IO, GT, 4, 96>), grid, dim3(256), 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (a.Dp) {
    case 32: hipLaunchKernelGGL((chunk_apply<IO, GT, 32>), grid, dim3(tpb), 0, s, a); break;
    case 64: hipLaunchKernelGGL((chunk_apply<IO, GT, 64>), grid, dim3(tpb), 0, s, a); break;
    case 96: hipLaunchKernelGGL((chunk_apply<IO, GT, 96>), grid, dim3(tpb), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template hipError_t launch_scan<float, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, bf16>(const ScanArgs&, hipStream_t);

}  // namespace holo
