// Device-side half of the CPU emulation of this package's gfx950 kernels:
// lane state, cross-lane collectives, matrix-core and buffer instructions.
// Test infrastructure only (see include/hip/hip_runtime.h).
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>

namespace emu {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

struct Dim { unsigned x, y, z; };

// ---- failures: print what and where, then abort the process ----
[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// ---- the running lane ----
struct Lane {
  Dim tid;
  int flat;        // linear thread index in the workgroup
  int wave;        // wave index in the workgroup
  int lane;        // lane index in the wave
};
extern Lane* g_lane;          // null in host code
extern Dim g_block_idx, g_block_dim, g_grid_dim;

inline Lane* cur() {
  if (!g_lane) fail("device function called outside a kernel launch");
  return g_lane;
}
inline const Dim& thread_idx() { return cur()->tid; }
inline const Dim& block_idx() { (void)cur(); return g_block_idx; }
inline const Dim& block_dim() { (void)cur(); return g_block_dim; }
inline const Dim& grid_dim() { (void)cur(); return g_grid_dim; }

void barrier();
void sleep_poll();
void waitcnt_vm(int n);
unsigned char* dyn_lds();

// ---- cross-lane collectives ----
// Each lane deposits up to 128 bytes; when every live lane of the wave has
// arrived at the same operation, `run` computes every lane's result (up to
// 64 bytes) from all deposits; each lane then takes its own.
enum OpKind : int { kOpShfl = 1, kOpBallot, kOpReadFirst, kOpPermSwap, kOpDsTr, kOpMfma };
struct WaveIO {
  alignas(64) unsigned char in[64][128];
  alignas(64) unsigned char out[64][64];
  uint64_t active;   // lanes that deposited
};
typedef void (*WaveRun)(WaveIO&);
// Deposits `in` (n_in bytes), waits for the wave, copies n_out bytes of this
// lane's result to `out`. `full` requires all 64 lanes (matrix cores and
// shuffles read every lane's registers).
void wave_collective(int kind, const void* site, WaveRun run, const void* in, size_t n_in, void* out, size_t n_out,
                     bool full);

template <typename T> struct ShflIn { T v; int src; };
template <typename T> void run_shfl(WaveIO& io) {
  for (int l = 0; l < 64; ++l) {
    if (!(io.active >> l & 1)) continue;
    ShflIn<T> s; std::memcpy(&s, io.in[l], sizeof s);
    ShflIn<T> t; std::memcpy(&t, io.in[s.src], sizeof t);
    std::memcpy(io.out[l], &t.v, sizeof(T));
  }
}
template <typename T> T shfl_src(T v, int src) {
  static_assert(sizeof(T) <= 8, "shuffle of at most 8 bytes");
  ShflIn<T> s{v, src};
  T r;
  wave_collective(kOpShfl, (const void*)&run_shfl<T>, &run_shfl<T>, &s, sizeof s, &r, sizeof r, true);
  return r;
}
template <typename T> T shfl_xor(T v, int m, int w) {
  const int self = cur()->lane;
  int idx = self ^ m;
  if (idx >= ((self + w) & ~(w - 1))) idx = self;
  return shfl_src(v, idx & 63);
}
template <typename T> T shfl_down(T v, unsigned d, int w) {
  const int self = cur()->lane;
  int idx = self + (int)d;
  if ((int)((self & (w - 1)) + d) >= w) idx = self;
  return shfl_src(v, idx);
}
template <typename T> T shfl(T v, int src, int w) {
  const int self = cur()->lane;
  return shfl_src(v, (src & (w - 1)) + (self & ~(w - 1)));
}

uint64_t ballot(bool p);
inline bool any(bool p) { return ballot(p) != 0; }
bool all(bool p);
int readfirstlane(int v);
u32x2 permlane32_swap(unsigned old, unsigned src, bool fi, bool bc);
s16x4 ds_read_tr16_b64(const void* p);

f32x16 mfma_32x32x2_f32(float a, float b, f32x16 c, int cbsz, int abid, int blgp);
f32x16 mfma_32x32x16_bf16(bf16x8 a, bf16x8 b, f32x16 c, int cbsz, int abid, int blgp);
f32x16 mfma_32x32x16_f16(f16x8 a, f16x8 b, f32x16 c, int cbsz, int abid, int blgp);

// dot products into fp32 (products of 16-bit values are exact in fp32; the
// two-term sum and the accumulator are rounded once, in double)
inline float fdot2_bf16(bf16x2 a, bf16x2 b, float c, bool) {
  return (float)((double)(float)a[0] * (double)(float)b[0] + (double)(float)a[1] * (double)(float)b[1] + (double)c);
}
inline float fdot2_f16(f16x2 a, f16x2 b, float c, bool) {
  return (float)((double)(float)a[0] * (double)(float)b[0] + (double)(float)a[1] * (double)(float)b[1] + (double)c);
}

// transcendental unit: the instructions' results to within their stated
// accuracy (1 ulp); the library functions are correctly rounded or nearly so
inline float exp2_f32(float x) { return std::exp2(x); }
inline float rcp_f32(float x) { return 1.0f / x; }
inline float rsq_f32(float x) { return 1.0f / std::sqrt(x); }

// ---- buffer resources ----
struct BufferRsrc {
  const unsigned char* base;
  uint32_t num_records;    // bytes (raw buffer: stride 0)
};
BufferRsrc make_buffer_rsrc(const void* p, int stride, int num_records, int flags);
// Copies `size` bytes at byte offset voffset + soffset + ioffset of the buffer
// into dst, each dword zero when it lies past num_records (the hardware's
// range check on the lane's offset). Fails when the two readings of that
// check (with or without the scalar offset) disagree for the access.
void buffer_read(const BufferRsrc& r, unsigned voffset, unsigned soffset, unsigned ioffset, void* dst, int size);
template <typename V> V buffer_load(const BufferRsrc& r, unsigned voffset, unsigned soffset, int aux) {
  (void)aux;
  V v;
  buffer_read(r, voffset, soffset, 0, &v, (int)sizeof(V));
  return v;
}
// buffer load whose data goes to LDS at lds + lane*size (lds wave-uniform),
// landing at this lane's next waitcnt_vm that covers it
void buffer_load_lds(const BufferRsrc& r, void* lds, unsigned size, unsigned voffset, unsigned soffset,
                     unsigned ioffset, unsigned aux);

// ---- atomics ----
template <typename T> T atomic_load(const T* p) { return __atomic_load_n(p, __ATOMIC_SEQ_CST); }
template <typename T, typename V> void atomic_store(T* p, V v) { __atomic_store_n(p, (T)v, __ATOMIC_SEQ_CST); }
template <typename T, typename V> T atomic_fetch_add(T* p, V v) { return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST); }
template <typename T, typename V> T atomic_fetch_or(T* p, V v) { return __atomic_fetch_or(p, (T)v, __ATOMIC_SEQ_CST); }

// ---- launches (host side) ----
void launch(const char* name, const void* fn, Dim grid, Dim block, size_t lds, std::function<void()> body);
bool take_launch_error();
void set_max_dynamic_lds(const void* fn, int bytes);
void host_copy(void* dst, const void* src, size_t n);

}  // namespace emu
