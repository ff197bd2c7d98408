// Attention dropout's keep mask on gfx950: the exact path's nn.Dropout on the
// softmax weights (kernel/attention_fast.py:160; core/attention.py:190),
// drawn from a counter-based generator so that the forward and each backward
// kernel regenerate the same mask from (seed, offset) without storing it.
//
// Generator: Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011). Each of its ten rounds takes the
// two 32x32->64-bit products M0 c0 and M1 c2 of the 128-bit counter and maps
//   (c0, c1, c2, c3) -> (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)),
// then adds the Weyl increments W0, W1 to the key.
//
// Pair (i, j) of head bh = b H + h is kept when word j % 4 of
//   philox4x32_10((i, j / 4, bh, offset), (seed mod 2^32, seed / 2^32))
// is >= thr = round(p 2^32); kept weights are scaled by 1 / (1 - p). A lane
// whose four consecutive keys share one query (the forward and dQ kernels'
// accumulator layout) uses all four words of one call.
#pragma once

#include "holo_kernels.h"

namespace holo {

__device__ __forceinline__ uint32_t mul_hi_u32(uint32_t a, uint32_t b) {
  return (uint32_t)(((uint64_t)a * (uint64_t)b) >> 32);
}

__device__ __forceinline__ u32x4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                               uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = mul_hi_u32(M0, c0), lo0 = M0 * c0;
    const uint32_t hi1 = mul_hi_u32(M1, c2), lo1 = M1 * c2;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  return u32x4{c0, c1, c2, c3};
}

// the random words of pairs (i, 4 j4 + e), e = 0..3, of head bh
__device__ __forceinline__ u32x4 keep_words(int64_t i, int64_t j4, int64_t bh, const DropParams& d) {
  return philox4x32_10((uint32_t)i, (uint32_t)j4, (uint32_t)bh, d.offset, d.k0, d.k1);
}

// element e of a 4-vector at a lane-dependent index (three selects)
__device__ __forceinline__ uint32_t pick4(const u32x4& v, int e) {
  const uint32_t lo = (e & 1) ? v[1] : v[0], hi = (e & 1) ? v[3] : v[2];
  return (e & 2) ? hi : lo;
}

}  // namespace holo
