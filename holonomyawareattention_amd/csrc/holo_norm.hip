// Residual add fused with LayerNorm for the decoder stack (gfx950).
//
// Reference behaviour (experiments/session_cherry.py:292-294): each pre-LN
// block computes h = h + core(ln1(h)), then ln2(h); across blocks the MLP's
// residual add is followed by the next block's ln1. One pass here:
//   h = x + delta                 (rounded to the storage dtype, as torch's add)
//   y = (h - mean(h)) / sqrt(var(h) + eps) * w + b     (nn.LayerNorm, biased
//                                 variance, statistics in fp32 from the rounded h)
// One wave per row: lane l owns the row's 16-byte chunks l, l + 64, ... and
// keeps them in registers; the mean and then the centred variance are wave
// reductions (two passes over registers, no second read of memory). Any d that
// is a multiple of 16 bytes, up to 64 * 16 chunks (8192 bf16, 4096 fp32).
#include "holo_kernels.h"

namespace holo {

template <typename T, int CH>
__global__ void __launch_bounds__(256) add_layernorm(AddNormArgs a) {
  constexpr int E = 16 / sizeof(T);                  // elements per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int nchunk = a.d / E;                        // chunks per row; lane owns lane + 64 c
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.n) return;                            // whole waves exit together
  const u32x4* xr = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.x) + row * a.x_rs);
  const u32x4* dr = reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.delta) + row * a.delta_rs);
  float v[CH * E];
  u32x4 xraw[CH], draw[CH];
  static_for<CH>([&](auto c) {
    const int ch = lane + 64 * c;
    if (ch < nchunk) { xraw[c] = xr[ch]; draw[c] = dr[ch]; }
    else { xraw[c] = u32x4{0, 0, 0, 0}; draw[c] = u32x4{0, 0, 0, 0}; }   // zeros: add nothing to the sum
  });
  float sum = 0.f;
  static_for<CH>([&](auto c) {
    const T* xe = reinterpret_cast<const T*>(&xraw[c]);
    const T* de = reinterpret_cast<const T*>(&draw[c]);
    static_for<E>([&](auto i) {
      const float hv = to_f32(from_f32<T>(to_f32(xe[i]) + to_f32(de[i])));   // h in its storage dtype
      v[c * E + i] = hv;
      sum += hv;
    });
  });
  static_for<6>([&](auto i) { sum += __shfl_xor(sum, 1 << (int)i); });
  const float inv_d = 1.f / (float)a.d;
  const float mean = sum * inv_d;
  float sq = 0.f;
  static_for<CH>([&](auto c) {
    const bool live = lane + 64 * c < nchunk;
    static_for<E>([&](auto i) {
      const float t = live ? v[c * E + i] - mean : 0.f;
      sq = __builtin_fmaf(t, t, sq);
    });
  });
  static_for<6>([&](auto i) { sq += __shfl_xor(sq, 1 << (int)i); });
  const float rstd = 1.f / sqrtf(sq * inv_d + a.eps);
  u32x4* hr = reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.h) + row * a.h_rs);
  u32x4* yr = reinterpret_cast<u32x4*>(reinterpret_cast<T*>(a.y) + row * a.y_rs);
  const u32x4* wr = reinterpret_cast<const u32x4*>(a.w);
  const u32x4* br = reinterpret_cast<const u32x4*>(a.b);
  static_for<CH>([&](auto c) {
    const int ch = lane + 64 * c;
    if (ch < nchunk) {
      const u32x4 wraw = wr[ch], braw = br[ch];
      const T* we = reinterpret_cast<const T*>(&wraw);
      const T* be = reinterpret_cast<const T*>(&braw);
      u32x4 hout, yout;
      T* ho = reinterpret_cast<T*>(&hout);
      T* yo = reinterpret_cast<T*>(&yout);
      static_for<E>([&](auto i) {
        const float hv = v[c * E + i];
        ho[i] = from_f32<T>(hv);
        yo[i] = from_f32<T>(__builtin_fmaf((hv - mean) * rstd, to_f32(we[i]), to_f32(be[i])));
      });
      hr[ch] = hout;
      yr[ch] = yout;
    }
  });
}

template <typename T>
hipError_t launch_add_layernorm(const AddNormArgs& a, hipStream_t s) {
  constexpr int E = 16 / sizeof(T);
  const dim3 grid((unsigned)((a.n + 3) / 4));
  const int ch = (a.d / E + 63) / 64;                // 16-byte chunks per lane
  if (a.d % E || ch > 16) return hipErrorInvalidValue;
  if (ch <= 1) hipLaunchKernelGGL((add_layernorm<T, 1>), grid, dim3(256), 0, s, a);
  else if (ch <= 2) hipLaunchKernelGGL((add_layernorm<T, 2>), grid, dim3(256), 0, s, a);
  else if (ch <= 3) hipLaunchKernelGGL((add_layernorm<T, 3>), grid, dim3(256), 0, s, a);
  else if (ch <= 4) hipLaunchKernelGGL((add_layernorm<T, 4>), grid, dim3(256), 0, s, a);
  else if (ch <= 6) hipLaunchKernelGGL((add_layernorm<T, 6>), grid, dim3(256), 0, s, a);
  else if (ch <= 8) hipLaunchKernelGGL((add_layernorm<T, 8>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((add_layernorm<T, 16>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template hipError_t launch_add_layernorm<float>(const AddNormArgs&, hipStream_t);
template hipError_t launch_add_layernorm<bf16>(const AddNormArgs&, hipStream_t);

}  // namespace holo
