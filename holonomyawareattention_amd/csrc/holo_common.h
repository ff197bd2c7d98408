// Shared device helpers for the gfx950 path-ordered attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace holo {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// fp16: the attention operands of the bf16 inference path (11-bit significand
// against bf16's 8, same matrix-core rate)
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// 16-byte and 8-byte raw moves: native vector types (HIP's uint4 is a union
// struct that is not split into registers when copied as an aggregate).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kChunk = 64;   // scan chunk = key tile = padding granule of T

// Compile-time loop: f(std::integral_constant<int, 0>{}) ... f(<N-1>{}), so that
// register arrays indexed by the loop variable never become stack arrays.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) { static_for_impl<0, N>(f); }

__host__ __device__ inline int padded_head_dim(int d) { return (d + 31) / 32 * 32; }
__host__ __device__ inline int64_t padded_seq(int64_t T) { return (T + kChunk - 1) / kChunk * kChunk; }

__device__ inline float to_f32(float x) { return x; }
__device__ inline float to_f32(bf16 x) { return (float)x; }
__device__ inline float to_f32(f16 x) { return (float)x; }
template <typename T> __device__ inline T from_f32(float x);
template <> __device__ inline float from_f32<float>(float x) { return x; }
template <> __device__ inline bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ inline f16 from_f32<f16>(float x) { return (f16)x; }

// Largest finite magnitude of a storage type (fp16 operands overflow to inf
// beyond it; the scan reports that in its status word).
template <typename T> constexpr float max_finite() { return 3.0e38f; }
template <> constexpr float max_finite<f16>() { return 65504.f; }

// Quaternion (w, x, y, z); R(a (x) b) = R(a) R(b).
struct quat { float w, x, y, z; };

// Explicit fused multiply-adds: the rounding of a product is the same
// wherever it is inlined (no context-dependent contraction), so a scan's
// result does not depend on how its carries are grouped.
__device__ inline quat qmul(const quat& a, const quat& b) {
  quat r;
  r.w = __builtin_fmaf(a.w, b.w, -__builtin_fmaf(a.x, b.x, __builtin_fmaf(a.y, b.y, a.z * b.z)));
  r.x = __builtin_fmaf(a.w, b.x, __builtin_fmaf(a.x, b.w, __builtin_fmaf(a.y, b.z, -(a.z * b.y))));
  r.y = __builtin_fmaf(a.w, b.y, __builtin_fmaf(-a.x, b.z, __builtin_fmaf(a.y, b.w, a.z * b.x)));
  r.z = __builtin_fmaf(a.w, b.z, __builtin_fmaf(a.x, b.y, __builtin_fmaf(-a.y, b.x, a.z * b.w)));
  return r;
}

__device__ inline quat qident() { return quat{1.f, 0.f, 0.f, 0.f}; }

// conjugate: the rotation of conj(q) is R(q)^T
__device__ inline quat qconj(const quat& q) { return quat{q.w, -q.x, -q.y, -q.z}; }

// exp of the skew block A = [[0,a0,a1],[-a0,0,a2],[-a1,-a2,0]]. A is the cross-
// product matrix of w = (-a2, a1, -a0), so exp(A) is the rotation by |w| about
// w: quaternion (cos(th/2), sin(th/2)/th * w). Below th = 1 both coefficients
// are their Taylor series in th^2 through th^8 (the first omitted terms are
// th^10 / 3.7e9 and th^10 / 8.2e10 of 1 and 1/2, below 3e-10 there): no
// square root, sine, cosine or division on the path every link takes at the
// generator scales of the reference's experiments.
__device__ inline quat qexp_skew(float a0, float a1, float a2) {
  float th2 = a0 * a0 + a1 * a1 + a2 * a2;
  float c, s;   // c = cos(th/2), s = sin(th/2)/th
  if (th2 < 1.f) {
    c = __builtin_fmaf(th2, __builtin_fmaf(th2, __builtin_fmaf(th2, __builtin_fmaf(th2, 1.f / 10321920.f,
                                                                                     -1.f / 46080.f),
                                                               1.f / 384.f),
                                           -0.125f),
                       1.f);
    s = __builtin_fmaf(th2, __builtin_fmaf(th2, __builtin_fmaf(th2, __builtin_fmaf(th2, 1.f / 185794560.f,
                                                                                     -1.f / 645120.f),
                                                               1.f / 3840.f),
                                           -1.f / 48.f),
                       0.5f);
  } else {
    float th = sqrtf(th2);
    float sh, ch;
    sincosf(0.5f * th, &sh, &ch);
    c = ch;
    s = sh / th;
  }
  return quat{c, -a2 * s, a1 * s, -a0 * s};
}

// Rotation matrix of q scaled by 1/|q|^2 (exactly orthogonal for any q != 0).
// These helpers spell out every fused multiply-add (fmaf) in a fixed order,
// so their rounding does not depend on how the compiler contracts the code
// around each inlined call: every kernel that rotates the same vector by the
// same quaternion gets the same bits.
struct rot3 { float m[3][3]; };

__device__ inline rot3 qmat(const quat& q) {
  const float zz = q.z * q.z;
  const float inv = __builtin_amdgcn_rcpf(fmaf(q.w, q.w, fmaf(q.x, q.x, fmaf(q.y, q.y, zz))));   // 1 ulp
  const float i2 = 2.f * inv;
  rot3 r;
  r.m[0][0] = fmaf(q.w, q.w, fmaf(q.x, q.x, -fmaf(q.y, q.y, zz))) * inv;
  r.m[0][1] = fmaf(q.x, q.y, -(q.w * q.z)) * i2;
  r.m[0][2] = fmaf(q.x, q.z, q.w * q.y) * i2;
  r.m[1][0] = fmaf(q.x, q.y, q.w * q.z) * i2;
  r.m[1][1] = fmaf(q.w, q.w, fmaf(q.y, q.y, -fmaf(q.x, q.x, zz))) * inv;
  r.m[1][2] = fmaf(q.y, q.z, -(q.w * q.x)) * i2;
  r.m[2][0] = fmaf(q.x, q.z, -(q.w * q.y)) * i2;
  r.m[2][1] = fmaf(q.y, q.z, q.w * q.x) * i2;
  r.m[2][2] = fmaf(q.w, q.w, fmaf(q.z, q.z, -fmaf(q.x, q.x, q.y * q.y))) * inv;
  return r;
}

// y = R^T u
__device__ inline void rot_t_apply(const rot3& R, float u0, float u1, float u2,
                                   float& y0, float& y1, float& y2) {
  y0 = fmaf(R.m[0][0], u0, fmaf(R.m[1][0], u1, R.m[2][0] * u2));
  y1 = fmaf(R.m[0][1], u0, fmaf(R.m[1][1], u1, R.m[2][1] * u2));
  y2 = fmaf(R.m[0][2], u0, fmaf(R.m[1][2], u1, R.m[2][2] * u2));
}

// y = R u
__device__ inline void rot_apply(const rot3& R, float u0, float u1, float u2,
                                 float& y0, float& y1, float& y2) {
  y0 = fmaf(R.m[0][0], u0, fmaf(R.m[0][1], u1, R.m[0][2] * u2));
  y1 = fmaf(R.m[1][0], u0, fmaf(R.m[1][1], u1, R.m[1][2] * u2));
  y2 = fmaf(R.m[2][0], u0, fmaf(R.m[2][1], u1, R.m[2][2] * u2));
}

// y = R(q) u with R the homogeneous rotation of q (same map as qmat):
// R(q) u = ((w^2 - |v|^2) u + 2 (v.u) v + 2 w (v x u)) / |q|^2,  v = (x, y, z)
__device__ inline void quat_rotate(const quat& q, float u0, float u1, float u2,
                                   float& y0, float& y1, float& y2) {
  const float vv = fmaf(q.x, q.x, fmaf(q.y, q.y, q.z * q.z));
  const float inv = __builtin_amdgcn_rcpf(fmaf(q.w, q.w, vv));
  const float a = fmaf(q.w, q.w, -vv) * inv;
  const float b = fmaf(q.x, u0, fmaf(q.y, u1, q.z * u2)) * (2.f * inv);
  const float cw = (2.f * q.w) * inv;
  y0 = fmaf(a, u0, fmaf(b, q.x, cw * fmaf(q.y, u2, -(q.z * u1))));
  y1 = fmaf(a, u1, fmaf(b, q.y, cw * fmaf(q.z, u0, -(q.x * u2))));
  y2 = fmaf(a, u2, fmaf(b, q.z, cw * fmaf(q.x, u1, -(q.y * u0))));
}

__device__ inline quat load_quat(const float* p) {
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  return quat{v[0], v[1], v[2], v[3]};
}

__device__ inline void store_quat(float* p, const quat& q) {
  f32x4 v = {q.w, q.x, q.y, q.z};
  *reinterpret_cast<f32x4*>(p) = v;
}

// Compact storage of a rotation: round(32767 * q / |q|) per component as
// int16, 8 bytes. |q / |q|| components are at most 1, so no value leaves
// [-32767, 32767].
__device__ inline void store_quat_snorm16(short* p, const quat& q) {
  const float s = 32767.f * __builtin_amdgcn_rsqf(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  auto cv = [&](float v) { return (unsigned)(int)__builtin_rintf(v * s) & 0xffffu; };
  *reinterpret_cast<u32x2*>(p) = u32x2{cv(q.w) | (cv(q.x) << 16), cv(q.y) | (cv(q.z) << 16)};
}

// store_quat_snorm16 with a non-temporal store (outputs streamed to HBM)
__device__ inline void store_quat_snorm16_nt(short* p, const quat& q) {
  const float s = 32767.f * __builtin_amdgcn_rsqf(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  auto cv = [&](float v) { return (unsigned)(int)__builtin_rintf(v * s) & 0xffffu; };
  __builtin_nontemporal_store(u32x2{cv(q.w) | (cv(q.x) << 16), cv(q.y) | (cv(q.z) << 16)}, reinterpret_cast<u32x2*>(p));
}

// The stored integers of store_quat_snorm16 as a quaternion (norm ~32767) of
// the same rotation: the homogeneous rotation map divides by |q|^2.
__device__ inline quat unpack_quat_snorm16(u32x2 v) {
  return quat{(float)(short)(v[0] & 0xffffu), (float)((int)v[0] >> 16),
              (float)(short)(v[1] & 0xffffu), (float)((int)v[1] >> 16)};
}

}  // namespace holo
