// Tile shapes and wave-level helpers shared by the attention kernels (gfx950).
#pragma once

#include <atomic>

#include "holo_kernels.h"

namespace holo {

constexpr int kBM = 128;                  // queries per workgroup
constexpr int kBN = 64;                   // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
// Running-max threshold (log2 units): the accumulator is rescaled only when a
// query's max grows by more than this, so exponentiated scores stay <= 2^8.
// Numerator and denominator use the same stale max, so the result is exact.
constexpr float kRescaleThreshold = 8.f;
// dword 3 of a raw buffer resource on gfx9-family targets (32-bit data format)
constexpr int kBufferWord3 = 0x00020000;

// max / sum of a value over lanes l and l^32 with a VALU lane swap (no LDS
// round trip): the two results of the swap hold the values of both halves
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float max3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

// maximum of the 32 scores a lane holds: a tree of 3-input maxima (16
// v_max3, depth 4) instead of a serial chain of dependent operations
__device__ __forceinline__ float tile_max(const f32x16 (&S)[2]) {
  float v[32], m[12];
  static_for<16>([&](auto r) { v[r] = S[0][(int)r]; v[16 + r] = S[1][(int)r]; });
  static_for<10>([&](auto i) { m[i] = max3(v[3 * i], v[3 * i + 1], v[3 * i + 2]); });
  m[10] = v[30]; m[11] = v[31];
  static_for<4>([&](auto i) { m[i] = max3(m[3 * i], m[3 * i + 1], m[3 * i + 2]); });
  return fmaxf(max3(m[0], m[1], m[2]), m[3]);
}

// Matrix-core operations of a 16-bit operand type on gfx950: the 32x32x16
// MFMA (fp32 accumulation) and the two-element dot product into fp32.
template <typename T> struct Op16;
template <> struct Op16<bf16> {
  typedef bf16x8 v8;
  typedef bf16x2 v2;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <> struct Op16<f16> {
  typedef f16x8 v8;
  typedef f16x2 v2;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
};

template <typename T, int DP> struct AttnCfg {
  static constexpr int E = 16 / sizeof(T);             // elements per 16 B
  // LDS row strides chosen so the MFMA operand reads hit distinct banks:
  // K rows (16 B per lane, 32 rows) at 52 dwords, V^T rows (8 B per lane,
  // 32 rows) at 34 dwords for bf16.
  static constexpr int KS = DP + E;
  static constexpr int VS = kBN + 4;
  static constexpr int OS = DP + 4;                     // fp32 staging
  static constexpr int NBX = (DP + 2) / 3;              // 3-dim groups covering DP
  static constexpr int KCH = kBN * DP / E / kThreads;   // 16 B chunks per thread per tile
  static constexpr int VCH = DP * kBN / E / kThreads;
  static constexpr int kStage = kBN * KS + DP * VS;     // elements of one K + V^T stage
  static constexpr int kStages = 3;
  static constexpr size_t kv_bytes = (size_t)kStages * kStage * sizeof(T);
  static constexpr size_t o_bytes = (size_t)kBM * OS * sizeof(float);
  static constexpr size_t lds = kv_bytes > o_bytes ? kv_bytes : o_bytes;
  static constexpr int NG8 = (NBX + 7) / 8;             // epilogue items per row (8 groups each)
  static constexpr int EPI = (kBM * NG8 + kThreads - 1) / kThreads;   // items per thread
  static_assert(KCH * E * kThreads == kBN * DP, "K tile must split evenly over the threads");
  static_assert(VCH * E * kThreads == kBN * DP, "V tile must split evenly over the threads");
  static_assert((kStage * sizeof(T)) % 16 == 0, "stages must stay 16-byte aligned");
};

typedef __attribute__((address_space(3))) void lds_void;

// Wait until at most N of this wave's vector memory operations (including
// buffer loads that write LDS) are outstanding.
template <int N> __device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier that also orders the LDS accesses around it for the compiler.
__device__ __forceinline__ void ring_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Largest dynamic LDS a workgroup may use on gfx950, and the device ids the
// opt-in below tracks.
constexpr int kMaxDynamicLds = 160 * 1024;
constexpr int kMaxDevices = 64;

// Opts `Kernel` into kMaxDynamicLds of dynamic LDS on the current device. The
// attribute belongs to the (kernel, device) pair, so it is set once per device
// that launches the kernel; launches then pass their own LDS size.
template <auto Kernel>
hipError_t allow_dynamic_lds() {
  static std::atomic<bool> done[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  if (done[dev].load(std::memory_order_acquire)) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kMaxDynamicLds);
  if (e == hipSuccess) done[dev].store(true, std::memory_order_release);
  return e;
}

}  // namespace holo
