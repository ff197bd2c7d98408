// CPU stand-in for <hip/hip_runtime.h>, used only to compile this package's
// gfx950 HIP sources for x86-64 (with AddressSanitizer) so that the kernels'
// own index arithmetic runs on the host, lane by lane, against bounds-checked
// memory. Test infrastructure: never part of the product library.
//
// Execution model (emu_runtime.cpp): every lane of a launch is a fiber; a
// workgroup's lanes run together, workgroups one after another in launch
// order. Cross-lane operations (MFMA, shuffles, ballots, LDS transposes, lane
// swaps) complete when every lane of the wave has reached them; buffer loads
// that write LDS land at the lane's next s_waitcnt that covers them, as the
// hardware's vmcnt orders them, so a tile read before its wait sees the
// previous contents.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>

#include "../emu_device.h"

// ---- qualifiers and attributes ----
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline __attribute__((always_inline))
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
#define __launch_bounds__(...)
#define address_space(n)
#define amdgpu_waves_per_eu(...) unused

// ---- indices ----
#define threadIdx (::emu::thread_idx())
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())

// ---- synchronisation ----
#define __syncthreads() ::emu::barrier()
#define __builtin_amdgcn_s_barrier() ::emu::barrier()
#define __builtin_amdgcn_s_sleep(n) ::emu::sleep_poll()

// ---- atomics (one host thread runs every lane: plain atomics suffice) ----
#define __HIP_MEMORY_SCOPE_AGENT 3
#define __HIP_MEMORY_SCOPE_WORKGROUP 2
#define __hip_atomic_load(p, o, s) ::emu::atomic_load((p))
#define __hip_atomic_store(p, v, o, s) ::emu::atomic_store((p), (v))
#define __hip_atomic_fetch_add(p, v, o, s) ::emu::atomic_fetch_add((p), (v))
#define __hip_atomic_fetch_or(p, v, o, s) ::emu::atomic_fetch_or((p), (v))

// ---- bit casts and math ----
__device__ inline float __uint_as_float(unsigned x) { float f; std::memcpy(&f, &x, 4); return f; }
__device__ inline unsigned __float_as_uint(float f) { unsigned x; std::memcpy(&x, &f, 4); return x; }
__device__ inline float __int_as_float(int x) { float f; std::memcpy(&f, &x, 4); return f; }
__device__ inline int __float_as_int(float f) { int x; std::memcpy(&x, &f, 4); return x; }
__device__ inline float __log2f(float x) { return std::log2(x); }
using std::fabs;

// ---- amdgcn builtins ----
#define __builtin_amdgcn_exp2f(x) ::emu::exp2_f32((x))
#define __builtin_amdgcn_rcpf(x) ::emu::rcp_f32((x))
#define __builtin_amdgcn_rsqf(x) ::emu::rsq_f32((x))
#define __builtin_amdgcn_readfirstlane(x) ::emu::readfirstlane((x))
#define __builtin_amdgcn_permlane32_swap(o, s, fi, bc) ::emu::permlane32_swap((o), (s), (fi), (bc))
#define __builtin_amdgcn_ds_read_tr16_b64_v4i16(p) ::emu::ds_read_tr16_b64((const void*)(p))
#define __builtin_amdgcn_fdot2_f32_bf16(a, b, c, cl) ::emu::fdot2_bf16((a), (b), (c), (cl))
#define __builtin_amdgcn_fdot2(a, b, c, cl) ::emu::fdot2_f16((a), (b), (c), (cl))
#define __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, x, y, z) ::emu::mfma_32x32x2_f32((a), (b), (c), (x), (y), (z))
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) ::emu::mfma_32x32x16_bf16((a), (b), (c), (x), (y), (z))
#define __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, x, y, z) ::emu::mfma_32x32x16_f16((a), (b), (c), (x), (y), (z))
typedef ::emu::BufferRsrc __amdgpu_buffer_rsrc_t;
#define __builtin_amdgcn_make_buffer_rsrc(p, st, n, fl) ::emu::make_buffer_rsrc((const void*)(p), (st), (n), (fl))
#define __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, aux) ::emu::buffer_load<::emu::u32x4>((r), (vo), (so), (aux))
#define __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, aux) ::emu::buffer_load<::emu::u32x2>((r), (vo), (so), (aux))
#define __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, aux) ::emu::buffer_load<unsigned>((r), (vo), (so), (aux))
#define __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, sz, vo, so, off, aux) \
  ::emu::buffer_load_lds((r), (void*)(lds), (sz), (vo), (so), (off), (aux))

// ---- HIP cross-lane functions ----
#define __ballot(p) ::emu::ballot((p))
#define __any(p) ::emu::any((p))
#define __all(p) ::emu::all((p))
template <typename T> __device__ inline T __shfl_xor(T v, int m, int w = 64) { return ::emu::shfl_xor(v, m, w); }
template <typename T> __device__ inline T __shfl_down(T v, unsigned d, int w = 64) { return ::emu::shfl_down(v, d, w); }
template <typename T> __device__ inline T __shfl(T v, int src, int w = 64) { return ::emu::shfl(v, src, w); }

// ---- host API (the subset the C ABI uses) ----
typedef enum hipError_t {
  hipSuccess = 0,
  hipErrorInvalidValue = 1,
  hipErrorInvalidDevice = 101,
  hipErrorLaunchFailure = 719,
} hipError_t;
typedef struct ihipStream_t* hipStream_t;
typedef enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyDefault = 4 } hipMemcpyKind;
typedef enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 } hipFuncAttribute;

struct dim3 {
  unsigned x, y, z;
  constexpr dim3(unsigned x_ = 1, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};

inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetLastError() { return ::emu::take_launch_error() ? hipErrorLaunchFailure : hipSuccess; }
inline const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "hipSuccess" : "emulated HIP error"; }
inline hipError_t hipFuncSetAttribute(const void* f, hipFuncAttribute attr, int value) {
  if (attr == hipFuncAttributeMaxDynamicSharedMemorySize) ::emu::set_max_dynamic_lds(f, value);
  return hipSuccess;
}
inline hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t) {
  ::emu::host_copy(dst, src, n);
  return hipSuccess;
}
#define HIP_SYMBOL(x) ((const void*)&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return hipSuccess; }

#define hipLaunchKernelGGL(K, G, B, L, S, ...)                                                         \
  ::emu::launch(#K, reinterpret_cast<const void*>(K), ::emu::Dim{dim3(G).x, dim3(G).y, dim3(G).z},      \
                ::emu::Dim{dim3(B).x, dim3(B).y, dim3(B).z}, (size_t)(L), [=]() { K(__VA_ARGS__); })
