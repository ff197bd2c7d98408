// Link rotations, chunked prefix-product scan and key/value transport (gfx950).
//
// Reference behaviour (core/attention_fast_chunked.py):
//   a_t   = edge_scale * (gq_t + gk_{(t+1) mod T})        additive   :80-84
//   (gq/gk are read in their own dtype GT, normally fp32, and composed in fp32)
//   a_t   = edge_scale * g_t                               direct a   :73-79
//   G_t   = exp(skew(a_t))                                 :86-87, core/utils.py:4-52
//   P_0 = I, P_{t+1} = G_t P_t ; Hol = G_{T-1} P_{T-1}     :89-95
//   kh_t  = P_t^T k_t,  vh_t = P_t^T v_t                    :109-110
//
// Each 3x3 block of every (b, h) is an independent scan over t. The scan runs
// in three launches over chunks of 64 links:
//   1. chunk_totals : one thread per (b, chunk, h, block) composes the chunk's
//                     64 link rotations (quaternions) into the chunk total;
//   2. chunk_carry  : one thread per (b, h, block) composes the totals in chunk
//                     order into exclusive carries (the prefix P at each chunk
//                     start) and the holonomy;
//   3. chunk_apply  : one thread per (b, chunk, h, block) starts from its
//                     carry, recomposes the chunk link by link, writes P_t and
//                     the transported kh, vh (zero padding included).
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

template <typename IO, typename GT>
__global__ void __launch_bounds__(256) chunk_apply(ScanArgs a) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t n = (int64_t)a.B * a.nch * a.H * a.nbx;
  if (gid >= n) return;
  int blk = gid % a.nbx;
  int h = (gid / a.nbx) % a.H;
  int64_t c = (gid / ((int64_t)a.nbx * a.H)) % a.nch;
  int b = gid / ((int64_t)a.nbx * a.H * a.nch);
  const int c0 = 3 * blk;
  int nc = a.Dp - c0; if (nc > 3) nc = 3;            // dims of this block inside Dp
  const int64_t bh = (int64_t)b * a.H + h;
  IO* kh = reinterpret_cast<IO*>(a.kh) + (bh * a.Tp + c * kChunk) * a.Dp + c0;
  IO* vt = reinterpret_cast<IO*>(a.vh_t) + ((bh * a.nch + c) * a.Dp + c0) * kChunk;
  const IO* kin = reinterpret_cast<const IO*>(a.k) + h * a.k_hs + c0;
  const IO* vin = reinterpret_cast<const IO*>(a.v) + h * a.v_hs + c0;
  const bool rot = blk < a.nb;
  quat p = rot ? load_quat(a.carry + (bh * a.nch + c) * a.nb * 4 + blk * 4) : qident();
  for (int i = 0; i < kChunk; ++i) {
    int64_t t = c * kChunk + i;
    float k3[3] = {0.f, 0.f, 0.f}, v3[3] = {0.f, 0.f, 0.f};
    if (t < a.T) {
      const IO* kr = kin + (b * a.T + t) * a.k_rs;
      const IO* vr = vin + (b * a.T + t) * a.v_rs;
      for (int j = 0; j < 3; ++j)
        if (c0 + j < a.d) { k3[j] = to_f32(kr[j]); v3[j] = to_f32(vr[j]); }
      if (rot) {
        store_quat(a.P + ((bh * a.T + t) * a.nb + blk) * 4, p);
        rot3 R = qmat(p);
        float y0, y1, y2;
        rot_t_apply(R, k3[0], k3[1], k3[2], y0, y1, y2);
        k3[0] = y0; k3[1] = y1; k3[2] = y2;
        rot_t_apply(R, v3[0], v3[1], v3[2], y0, y1, y2);
        v3[0] = y0; v3[1] = y1; v3[2] = y2;
        if (t + 1 < a.T) p = qmul(link_quat<GT>(a, b, h, blk, t), p);
      }
    }
    for (int j = 0; j < nc; ++j) {
      kh[(int64_t)i * a.Dp + j] = from_f32<IO>(k3[j]);
      vt[(int64_t)j * kChunk + i] = from_f32<IO>(v3[j]);
    }
  }
}

template <typename IO, typename GT>
hipError_t launch_scan(const ScanArgs& a, hipStream_t s) {
  const int tpb = 256;
  int64_t n1 = (int64_t)a.B * a.nch * a.H * a.nb;
  int64_t n2 = (int64_t)a.B * a.H * a.nb;
  int64_t n3 = (int64_t)a.B * a.nch * a.H * a.nbx;
  if (n1 > 0) hipLaunchKernelGGL(chunk_totals<GT>, dim3((n1 + tpb - 1) / tpb), dim3(tpb), 0, s, a);
  if (n2 > 0) hipLaunchKernelGGL(chunk_carry<GT>, dim3((n2 + tpb - 1) / tpb), dim3(tpb), 0, s, a);
  hipLaunchKernelGGL((chunk_apply<IO, GT>), dim3((n3 + tpb - 1) / tpb), dim3(tpb), 0, s, a);
  return hipGetLastError();
}

template hipError_t launch_scan<float, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, float>(const ScanArgs&, hipStream_t);
template hipError_t launch_scan<bf16, bf16>(const ScanArgs&, hipStream_t);

}  // namespace holo
