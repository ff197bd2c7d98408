// Chained state shared by the single-pass scans (forward prefix products and
// the backward's suffix sums): per-(b, h, chunk) 16-byte slots whose 32-bit
// words start unset and are written once per launch.
#pragma once

#include "holo_common.h"

namespace holo {

// A slot (four fp32 words: a quaternion, or a 3-vector and a pad word, per
// (b, h, chunk, block)) starts with every word kUnset. Each word is written
// once per launch and read with agent-scope relaxed atomics, so a word is
// either unset or final and readers need no fence: a slot is complete when
// none of its words is unset. A computed word equal to kUnset (one NaN bit
// pattern) is stored as the canonical NaN instead.
constexpr unsigned kUnset = 0xffffffffu;
constexpr unsigned kCanonNan = 0x7fc00000u;
constexpr int kMaxPolls = 1 << 18;   // ~0.3 s of polling
// Bits of the status word that follows the ticket counter in a chained
// workspace (cleared by the reset launch at the start of every call).
constexpr unsigned kStatusTimeout = 1u;    // a carry wait ran out of polls (outputs NaN)
constexpr unsigned kStatusOverflow = 2u;   // a transported value exceeded the operand type's range

__device__ __forceinline__ void put_quat(float* slot, const quat& q) {
  unsigned* u = reinterpret_cast<unsigned*>(slot);
  const float v[4] = {q.w, q.x, q.y, q.z};
  static_for<4>([&](auto k) {
    unsigned x = __float_as_uint(v[k]);
    if (x == kUnset) x = kCanonNan;
    __hip_atomic_store(u + k, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  });
}

__device__ __forceinline__ bool get_quat(const float* slot, quat& q) {
  const unsigned* u = reinterpret_cast<const unsigned*>(slot);
  unsigned x[4];
  static_for<4>([&](auto k) { x[k] = __hip_atomic_load(u + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); });
  if (x[0] == kUnset || x[1] == kUnset || x[2] == kUnset || x[3] == kUnset) return false;
  q = quat{__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3])};
  return true;
}

}  // namespace holo
