// Host runtime of the CPU emulation of this package's gfx950 kernels (test
// infrastructure only): fibers for lanes, the workgroup scheduler, wave
// collectives, matrix-core and buffer-instruction semantics, and guarded
// allocations against which every global access is bounds-checked.
//
// Memory checks:
//  - emu_alloc places each buffer at the start of a read/write region that is
//    flanked by 64 MiB of inaccessible address space on both sides; the bytes
//    between the buffer's end and the end of its last page are poisoned for
//    AddressSanitizer. Any load or store outside the buffer therefore stops
//    the process with a report naming the kernel source line.
//  - A buffer resource's range [base, base + num_records) must lie inside one
//    registered allocation (the hardware may fetch anywhere in that range).
//  - Dynamic LDS is a guarded region of exactly the launch's LDS bytes, filled
//    with a marker pattern before every workgroup; static __shared__ arrays are
//    globals with AddressSanitizer redzones.
//  - A launch with more dynamic LDS than 64 KiB needs the kernel's
//    hipFuncAttributeMaxDynamicSharedMemorySize opt-in, and at most 160 KiB.
#include "emu_device.h"

#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#include <sys/mman.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

extern "C" void emu_ctx_switch(void** save_sp, void* load_sp);
// Saves the callee-saved registers, the x87 control word and MXCSR on the
// current stack, stores the stack pointer to *save_sp and resumes the context
// whose stack pointer is load_sp (System V x86-64).
asm(R"(
.text
.globl emu_ctx_switch
.type emu_ctx_switch, @function
emu_ctx_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    subq $16, %rsp
    stmxcsr 8(%rsp)
    fnstcw (%rsp)
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    fldcw (%rsp)
    ldmxcsr 8(%rsp)
    addq $16, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
.size emu_ctx_switch, .-emu_ctx_switch
)");

namespace emu {

Lane* g_lane = nullptr;
Dim g_block_idx{0, 0, 0}, g_block_dim{1, 1, 1}, g_grid_dim{1, 1, 1};

namespace {

constexpr size_t kGuard = (size_t)64 << 20;
constexpr size_t kPage = 4096;
constexpr size_t kStack = (size_t)256 << 10;
constexpr int kMaxThreads = 1024;
constexpr size_t kMaxLds = 160 * 1024;
constexpr size_t kDefaultLds = 64 * 1024;
constexpr int kMaxPending = 63;     // vmcnt saturates at 63 outstanding operations per wave

// ---- allocations ----
struct Alloc { uintptr_t base; size_t size; void* map; size_t map_size; };
std::map<uintptr_t, Alloc> g_allocs;   // by base

const Alloc* find_alloc(uintptr_t p) {
  auto it = g_allocs.upper_bound(p);
  if (it == g_allocs.begin()) return nullptr;
  --it;
  const Alloc& a = it->second;
  if (p >= a.base && p <= a.base + a.size) return &a;   // one past the end counts (empty ranges)
  return nullptr;
}

void* guarded_map(size_t n, Alloc& a) {
  const size_t body = (n + kPage - 1) / kPage * kPage + (n % kPage == 0 ? kPage : 0);
  a.map_size = kGuard + body + kGuard;
  void* m = mmap(nullptr, a.map_size, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  if (m == MAP_FAILED) return nullptr;
  unsigned char* b = static_cast<unsigned char*>(m) + kGuard;
  if (mprotect(b, body, PROT_READ | PROT_WRITE) != 0) { munmap(m, a.map_size); return nullptr; }
  a.map = m;
  a.base = reinterpret_cast<uintptr_t>(b);
  a.size = n;
  __asan_poison_memory_region(b + n, body - n);   // the tail of the last page
  return b;
}

// ---- launch configuration and statistics ----
std::unordered_map<const void*, int> g_max_dyn_lds;
bool g_launch_error = false;
int64_t g_sample_head = 0, g_sample_tail = 0, g_sample_stride = 0;   // 0, 0, 0: every workgroup
int g_lds_dma_mode = 0;    // 0: LDS-DMA data lands at the covering waitcnt; 1: at issue
bool g_log = false;
std::string g_log_text;
int64_t g_stats[16];
enum Stat { kLaunches, kBlocks, kLanes, kCollectives, kMfma, kLdsDma, kPartialDword, kPolls, kBufLoads, kNStats };
const char* g_launch_name = "";

// ---- fibers ----
enum Wait : int { kRun = 0, kWave, kBar, kDone };
struct Pending { unsigned char* dst; int size; unsigned char data[16]; };
struct Fiber {
  Lane lane;
  void* sp;
  unsigned char* stack;
  int wait;
  uint64_t wait_gen;
  Pending pend[kMaxPending];
  int npend, pend_head;
  void* fake;            // AddressSanitizer fake-stack slot of this fiber
  int64_t dma_issued;    // LDS-DMA instructions issued by this lane (uniformity check index)
};
struct Wave {
  int nlanes, live, arrived;
  uint64_t gen;
  uint64_t lanes_mask;
  int kind;
  WaveRun run;
  bool full;
  WaveIO io;
  int64_t dma_idx[64];
  const void* dma_base[64];
};
struct Block {
  int nthreads, live, bar_arrived;
  uint64_t bar_gen;
  std::vector<Wave> waves;
};

unsigned char* g_stacks = nullptr;
Fiber* g_fibers = nullptr;
Fiber* g_cur = nullptr;
Block g_blk;
void* g_sched_sp = nullptr;
void* g_sched_fake = nullptr;
const void* g_main_bottom = nullptr;
size_t g_main_size = 0;
const std::function<void()>* g_body = nullptr;
unsigned char* g_dyn_lds = nullptr;
size_t g_dyn_lds_bytes = 0;
unsigned g_fpcw = 0x037f, g_mxcsr = 0x1f80;

void fiber_entry();

void init_stacks() {
  if (g_stacks) return;
  const size_t total = (size_t)kMaxThreads * kStack;
  void* m = mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  if (m == MAP_FAILED) fail("cannot map %zu bytes of lane stacks", total);
  g_stacks = static_cast<unsigned char*>(m);
  for (int i = 0; i < kMaxThreads; ++i) mprotect(g_stacks + (size_t)i * kStack, kPage, PROT_NONE);   // overflow guard
  g_fibers = new Fiber[kMaxThreads];
}

void init_fiber(Fiber& f, int i) {
  f.stack = g_stacks + (size_t)i * kStack;
  unsigned char* top = f.stack + kStack;                    // 16-byte aligned
  uint64_t* s = reinterpret_cast<uint64_t*>(top);
  s[-1] = 0;                                                // fake return address of fiber_entry
  s[-2] = reinterpret_cast<uint64_t>(&fiber_entry);
  for (int k = 3; k <= 8; ++k) s[-k] = 0;                   // rbp rbx r12 r13 r14 r15
  s[-10] = g_fpcw;                                          // x87 control word at sp
  s[-9] = g_mxcsr;                                          // MXCSR at sp + 8
  f.sp = top - 80;
  f.wait = kRun;
  f.wait_gen = 0;
  f.npend = 0;
  f.pend_head = 0;
  f.dma_issued = 0;
  f.fake = nullptr;
}

void switch_to(Fiber& f) {
  g_cur = &f;
  g_lane = &f.lane;
  __sanitizer_start_switch_fiber(&g_sched_fake, f.stack + kPage, kStack - kPage);
  emu_ctx_switch(&g_sched_sp, f.sp);
  __sanitizer_finish_switch_fiber(g_sched_fake, nullptr, nullptr);
  g_lane = nullptr;
  g_cur = nullptr;
}

void to_scheduler(Fiber& f, bool dying) {
  __sanitizer_start_switch_fiber(dying ? nullptr : &f.fake, g_main_bottom, g_main_size);
  emu_ctx_switch(&f.sp, g_sched_sp);
  __sanitizer_finish_switch_fiber(f.fake, nullptr, nullptr);
  if (dying) fail("a finished lane was resumed");
  g_cur = &f;
  g_lane = &f.lane;
}

void apply_pending(Fiber& f, int keep) {
  while (f.npend > keep) {
    Pending& p = f.pend[f.pend_head];
    std::memcpy(p.dst, p.data, p.size);
    f.pend_head = (f.pend_head + 1) % kMaxPending;
    --f.npend;
  }
}

void complete_wave(Wave& w) {
  if (w.full && w.io.active != w.lanes_mask)
    fail("a cross-lane operation (kind %d) needs every lane of the wave; active lanes 0x%016llx of 0x%016llx",
         w.kind, (unsigned long long)w.io.active, (unsigned long long)w.lanes_mask);
  w.run(w.io);
  w.arrived = 0;
  ++w.gen;
  ++g_stats[kCollectives];
}

void lane_exit(Fiber& f) {
  apply_pending(f, 0);
  Wave& w = g_blk.waves[f.lane.wave];
  --g_blk.live;
  --w.live;
  if (w.arrived > 0 && w.arrived == w.live) complete_wave(w);
  if (g_blk.bar_arrived > 0 && g_blk.bar_arrived == g_blk.live) {
    g_blk.bar_arrived = 0;
    ++g_blk.bar_gen;
  }
}

void fiber_entry() {
  Fiber& f = *g_cur;
  __sanitizer_finish_switch_fiber(nullptr, &g_main_bottom, &g_main_size);
  (*g_body)();
  lane_exit(f);
  f.wait = kDone;
  to_scheduler(f, true);
  __builtin_unreachable();
}

void deadlock() {
  std::string s;
  char buf[256];
  snprintf(buf, sizeof buf, "workgroup barrier: %d of %d live lanes arrived; ", g_blk.bar_arrived, g_blk.live);
  s += buf;
  for (size_t i = 0; i < g_blk.waves.size(); ++i) {
    const Wave& w = g_blk.waves[i];
    if (w.arrived) {
      snprintf(buf, sizeof buf, "wave %zu: %d of %d lanes at a cross-lane op (kind %d); ", i, w.arrived, w.live, w.kind);
      s += buf;
    }
  }
  fail("deadlock: %s", s.c_str());
}

void run_block() {
  const int n = g_blk.nthreads;
  for (int i = 0; i < n; ++i) {
    Fiber& f = g_fibers[i];
    init_fiber(f, i);
    const unsigned bx = g_block_dim.x, by = g_block_dim.y;
    f.lane.tid = Dim{(unsigned)i % bx, ((unsigned)i / bx) % by, (unsigned)i / (bx * by)};
    f.lane.flat = i;
    f.lane.wave = i / 64;
    f.lane.lane = i % 64;
  }
  const int nw = (n + 63) / 64;
  g_blk.waves.assign(nw, Wave{});
  for (int wi = 0; wi < nw; ++wi) {
    Wave& w = g_blk.waves[wi];
    w.nlanes = (wi + 1) * 64 <= n ? 64 : n - wi * 64;
    w.live = w.nlanes;
    w.lanes_mask = w.nlanes == 64 ? ~0ull : ((1ull << w.nlanes) - 1);
    for (int k = 0; k < 64; ++k) w.dma_idx[k] = -1;
  }
  g_blk.live = n;
  g_blk.bar_arrived = 0;
  g_blk.bar_gen = 0;
  if (g_dyn_lds) std::memset(g_dyn_lds, 0xee, g_dyn_lds_bytes);
  while (g_blk.live > 0) {
    bool progressed = false;
    for (int i = 0; i < n; ++i) {
      Fiber& f = g_fibers[i];
      if (f.wait == kDone) continue;
      if (f.wait == kWave && g_blk.waves[f.lane.wave].gen == f.wait_gen) continue;
      if (f.wait == kBar && g_blk.bar_gen == f.wait_gen) continue;
      f.wait = kRun;
      progressed = true;
      switch_to(f);
    }
    if (!progressed) deadlock();
  }
  g_stats[kBlocks] += 1;
  g_stats[kLanes] += n;
}

bool sampled(int64_t b, int64_t total) {
  if (g_sample_head == 0 && g_sample_tail == 0 && g_sample_stride == 0) return true;
  if (b < g_sample_head || b >= total - g_sample_tail) return true;
  return g_sample_stride > 0 && b % g_sample_stride == 0;
}

}  // namespace

void fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fprintf(stderr, "EMU FAILURE: ");
  vfprintf(stderr, fmt, ap);
  va_end(ap);
  if (g_lane)
    fprintf(stderr, "\n  in launch %s, workgroup (%u, %u, %u) of (%u, %u, %u), thread %d (wave %d, lane %d)\n",
            g_launch_name, g_block_idx.x, g_block_idx.y, g_block_idx.z, g_grid_dim.x, g_grid_dim.y, g_grid_dim.z,
            g_lane->flat, g_lane->wave, g_lane->lane);
  else
    fprintf(stderr, "\n  (host side, last launch %s)\n", g_launch_name);
  fflush(stderr);
  abort();
}

// ---- device functions ----
void barrier() {
  Fiber& f = *g_cur;
  ++g_blk.bar_arrived;
  if (g_blk.bar_arrived == g_blk.live) {
    g_blk.bar_arrived = 0;
    ++g_blk.bar_gen;
    return;
  }
  f.wait = kBar;
  f.wait_gen = g_blk.bar_gen;
  to_scheduler(f, false);
}

void sleep_poll() {
  Fiber& f = *g_cur;
  ++g_stats[kPolls];
  f.wait = kRun;
  to_scheduler(f, false);
}

void waitcnt_vm(int n) { apply_pending(*g_cur, n < 0 ? 0 : n); }

unsigned char* dyn_lds() {
  if (!g_dyn_lds) fail("kernel uses dynamic LDS but the launch requested none");
  return g_dyn_lds;
}

void wave_collective(int kind, const void* site, WaveRun run, const void* in, size_t n_in, void* out, size_t n_out,
                     bool full) {
  (void)site;
  Fiber& f = *g_cur;
  Wave& w = g_blk.waves[f.lane.wave];
  if (w.arrived == 0) {
    w.kind = kind;
    w.run = run;
    w.full = full;
    w.io.active = 0;
  } else if (w.kind != kind || w.run != run) {
    fail("divergent cross-lane operations in one wave (kinds %d and %d)", w.kind, kind);
  }
  std::memcpy(w.io.in[f.lane.lane], in, n_in);
  w.io.active |= 1ull << f.lane.lane;
  ++w.arrived;
  if (w.arrived == w.live) {
    complete_wave(w);
  } else {
    f.wait = kWave;
    f.wait_gen = w.gen;
    to_scheduler(f, false);
  }
  std::memcpy(out, w.io.out[f.lane.lane], n_out);
}

namespace {
void run_ballot(WaveIO& io) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((io.active >> l & 1) && io.in[l][0]) m |= 1ull << l;
  for (int l = 0; l < 64; ++l) std::memcpy(io.out[l], &m, 8);
}
void run_readfirst(WaveIO& io) {
  int first = __builtin_ctzll(io.active);
  for (int l = 0; l < 64; ++l) std::memcpy(io.out[l], io.in[first], 4);
}
void run_permswap(WaveIO& io) {
  // v_permlane32_swap: lanes 32..63 of the first operand trade places with
  // lanes 0..31 of the second
  for (int l = 0; l < 64; ++l) {
    unsigned o[2], r[2];
    std::memcpy(o, io.in[l], 8);
    if (l < 32) {
      unsigned hi[2]; std::memcpy(hi, io.in[l + 32], 8);
      r[0] = o[0];
      r[1] = hi[0];
    } else {
      unsigned lo[2]; std::memcpy(lo, io.in[l - 32], 8);
      r[0] = lo[1];
      r[1] = o[1];
    }
    std::memcpy(io.out[l], r, 8);
  }
}
void run_ds_tr16(WaveIO& io) {
  // ds_read_b64_tr_b16: lane i of each 16-lane group receives element i % 4
  // of the 4-element reads of the group's lanes i / 4 + {0, 4, 8, 12}
  for (int l = 0; l < 64; ++l) {
    const int G = l >> 4, i = l & 15;
    short r[4];
    for (int e = 0; e < 4; ++e) {
      short src[4];
      std::memcpy(src, io.in[G * 16 + i / 4 + 4 * e], 8);
      r[e] = src[i % 4];
    }
    std::memcpy(io.out[l], r, 8);
  }
}
// 32x32 output layout of the 32x32xK MFMAs: lane l, register r holds
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
inline int mfma_row(int l, int r) { return 8 * (r / 4) + 4 * (l / 32) + (r % 4); }
template <int K, typename Elem> void run_mfma(WaveIO& io) {
  // operand layout: lane l holds A[l % 32][(K / 2) (l / 32) + e] and
  // B[(K / 2) (l / 32) + e][l % 32], e < K / 2 (K = 2: one element each)
  constexpr int H = K / 2;
  double A[32][K], Bm[K][32], D[32][32];
  for (int l = 0; l < 64; ++l) {
    Elem a[H], b[H];
    float c[16];
    std::memcpy(a, io.in[l], sizeof a);
    std::memcpy(b, io.in[l] + 16, sizeof b);
    std::memcpy(c, io.in[l] + 32, sizeof c);
    for (int e = 0; e < H; ++e) {
      A[l % 32][H * (l / 32) + e] = (double)(float)a[e];
      Bm[H * (l / 32) + e][l % 32] = (double)(float)b[e];
    }
    for (int r = 0; r < 16; ++r) D[mfma_row(l, r)][l % 32] = c[r];
  }
  for (int i = 0; i < 32; ++i)
    for (int j = 0; j < 32; ++j) {
      double s = D[i][j];
      for (int k = 0; k < K; ++k) s += A[i][k] * Bm[k][j];
      D[i][j] = s;
    }
  for (int l = 0; l < 64; ++l) {
    float d[16];
    for (int r = 0; r < 16; ++r) d[r] = (float)D[mfma_row(l, r)][l % 32];
    std::memcpy(io.out[l], d, sizeof d);
  }
  ++g_stats[kMfma];
}
template <typename AV, typename BV>
f32x16 mfma_call(WaveRun run, const AV& a, const BV& b, const f32x16& c, int cbsz, int abid, int blgp) {
  if (cbsz || abid || blgp) fail("MFMA broadcast/swizzle modifiers are not modelled (cbsz %d abid %d blgp %d)", cbsz, abid, blgp);
  unsigned char in[96] = {};
  std::memcpy(in, &a, sizeof a);
  std::memcpy(in + 16, &b, sizeof b);
  std::memcpy(in + 32, &c, 64);
  f32x16 d;
  wave_collective(kOpMfma, (const void*)run, run, in, sizeof in, &d, sizeof d, true);
  return d;
}
}  // namespace

uint64_t ballot(bool p) {
  unsigned char in = p ? 1 : 0;
  uint64_t r;
  wave_collective(kOpBallot, (const void*)&run_ballot, &run_ballot, &in, 1, &r, 8, false);
  return r;
}
bool all(bool p) {
  const uint64_t m = ballot(p);
  return m == g_blk.waves[g_cur->lane.wave].io.active;
}
int readfirstlane(int v) {
  int r;
  wave_collective(kOpReadFirst, (const void*)&run_readfirst, &run_readfirst, &v, 4, &r, 4, false);
  return r;
}
u32x2 permlane32_swap(unsigned old, unsigned src, bool fi, bool bc) {
  if (fi || bc) fail("permlane32_swap with fetch-inactive or bound-control set is not modelled");
  unsigned in[2] = {old, src};
  u32x2 r;
  wave_collective(kOpPermSwap, (const void*)&run_permswap, &run_permswap, in, 8, &r, 8, true);
  return r;
}
s16x4 ds_read_tr16_b64(const void* p) {
  s16x4 v;
  std::memcpy(&v, p, 8);      // the lane's own 8-byte LDS read (bounds-checked here)
  s16x4 r;
  wave_collective(kOpDsTr, (const void*)&run_ds_tr16, &run_ds_tr16, &v, 8, &r, 8, true);
  return r;
}
f32x16 mfma_32x32x2_f32(float a, float b, f32x16 c, int cbsz, int abid, int blgp) {
  return mfma_call(&run_mfma<2, float>, a, b, c, cbsz, abid, blgp);
}
f32x16 mfma_32x32x16_bf16(bf16x8 a, bf16x8 b, f32x16 c, int cbsz, int abid, int blgp) {
  return mfma_call(&run_mfma<16, __bf16>, a, b, c, cbsz, abid, blgp);
}
f32x16 mfma_32x32x16_f16(f16x8 a, f16x8 b, f32x16 c, int cbsz, int abid, int blgp) {
  return mfma_call(&run_mfma<16, _Float16>, a, b, c, cbsz, abid, blgp);
}

// ---- buffer instructions ----
BufferRsrc make_buffer_rsrc(const void* p, int stride, int num_records, int flags) {
  if (stride != 0) fail("buffer resource with stride %d (only raw buffers are modelled)", stride);
  if (flags != 0x00020000) fail("buffer resource dword 3 0x%08x (expected the 32-bit raw format 0x00020000)", flags);
  if (num_records < 0) fail("buffer resource of %d bytes: the 32-bit record count overflowed", num_records);
  const uintptr_t b = reinterpret_cast<uintptr_t>(p);
  const Alloc* a = find_alloc(b);
  if (num_records > 0) {
    if (!a) fail("buffer resource base %p lies in no allocation", p);
    if (b + (uintptr_t)num_records > a->base + a->size)
      fail("buffer resource [%p, +%d) ends %lld bytes past its allocation [%p, +%zu)", p, num_records,
           (long long)(b + num_records - a->base - a->size), (void*)a->base, a->size);
  }
  return BufferRsrc{static_cast<const unsigned char*>(p), (uint32_t)num_records};
}

void buffer_read(const BufferRsrc& r, unsigned voffset, unsigned soffset, unsigned ioffset, void* dst, int size) {
  ++g_stats[kBufLoads];
  unsigned char* d = static_cast<unsigned char*>(dst);
  int in_count = 0;
  for (int i = 0; i < size; i += 4) {
    const uint64_t off_v = (uint64_t)voffset + ioffset + i;
    const uint64_t off_f = off_v + soffset;
    const bool in_v = off_v + 4 <= r.num_records, in_f = off_f + 4 <= r.num_records;
    if (in_v != in_f)
      fail("buffer load at voffset %u + soffset %u + %d: in range only %s the scalar offset (num_records %u)", voffset,
           soffset, i, in_f ? "with" : "without", r.num_records);
    if (in_f) {
      std::memcpy(d + i, r.base + off_f, 4);
      ++in_count;
    } else {
      std::memset(d + i, 0, 4);
    }
  }
  if (in_count != 0 && in_count != size / 4) ++g_stats[kPartialDword];
}

void buffer_load_lds(const BufferRsrc& r, void* lds, unsigned size, unsigned voffset, unsigned soffset,
                     unsigned ioffset, unsigned aux) {
  (void)aux;
  if (ioffset != 0) fail("buffer load to LDS with an instruction offset (%u) is not modelled", ioffset);
  if (size != 4 && size != 12 && size != 16) fail("buffer load to LDS of %u bytes", size);
  Fiber& f = *g_cur;
  Wave& w = g_blk.waves[f.lane.wave];
  // the LDS base is a scalar (M0): every lane of the wave must pass the same
  const int slot = (int)(f.dma_issued & 63);
  if (w.dma_idx[slot] == f.dma_issued) {
    if (w.dma_base[slot] != lds) fail("buffer load to LDS with a lane-varying LDS base");
  } else {
    w.dma_idx[slot] = f.dma_issued;
    w.dma_base[slot] = lds;
  }
  ++f.dma_issued;
  ++g_stats[kLdsDma];
  unsigned char* dst = static_cast<unsigned char*>(lds) + (size_t)f.lane.lane * size;
  unsigned char data[16];
  buffer_read(r, voffset, soffset, 0, data, (int)size);
  if (g_lds_dma_mode == 1) {
    std::memcpy(dst, data, size);
    return;
  }
  if (f.npend == kMaxPending) apply_pending(f, kMaxPending - 1);
  Pending& p = f.pend[(f.pend_head + f.npend) % kMaxPending];
  p.dst = dst;
  p.size = (int)size;
  std::memcpy(p.data, data, size);
  ++f.npend;
}

// ---- host side ----
void set_max_dynamic_lds(const void* fn, int bytes) { g_max_dyn_lds[fn] = bytes; }
bool take_launch_error() { bool e = g_launch_error; g_launch_error = false; return e; }
void host_copy(void* dst, const void* src, size_t n) { std::memmove(dst, src, n); }

void launch(const char* name, const void* fn, Dim grid, Dim block, size_t lds, std::function<void()> body) {
  g_launch_name = name;
  const int64_t nthreads = (int64_t)block.x * block.y * block.z;
  if (nthreads < 1 || nthreads > kMaxThreads) fail("workgroup of %lld threads", (long long)nthreads);
  const int64_t total = (int64_t)grid.x * grid.y * grid.z;
  if (total < 1) fail("empty grid (%u, %u, %u)", grid.x, grid.y, grid.z);
  if (grid.y > 65535 || grid.z > 65535 || grid.x > 0x7fffffffu) fail("grid (%u, %u, %u) beyond the limits", grid.x, grid.y, grid.z);
  if (lds > kMaxLds) fail("%zu bytes of dynamic LDS (at most %zu)", lds, kMaxLds);
  if (lds > kDefaultLds) {
    auto it = g_max_dyn_lds.find(fn);
    if (it == g_max_dyn_lds.end() || (size_t)it->second < lds)
      fail("%zu bytes of dynamic LDS without the kernel's opt-in beyond %zu", lds, kDefaultLds);
  }
  if (g_log) {
    char buf[512];
    snprintf(buf, sizeof buf, "%s grid=(%u,%u,%u) block=(%u,%u,%u) lds=%zu\n", name, grid.x, grid.y, grid.z, block.x,
             block.y, block.z, lds);
    g_log_text += buf;
  }
  ++g_stats[kLaunches];
  init_stacks();
  {
    unsigned short cw;
    unsigned mx;
    asm volatile("fnstcw %0" : "=m"(cw));
    asm volatile("stmxcsr %0" : "=m"(mx));
    g_fpcw = cw;
    g_mxcsr = mx;
  }
  Alloc lds_alloc{};
  g_dyn_lds = nullptr;
  g_dyn_lds_bytes = lds;
  if (lds > 0) {
    g_dyn_lds = static_cast<unsigned char*>(guarded_map(lds, lds_alloc));
    if (!g_dyn_lds) fail("cannot map %zu bytes of LDS", lds);
  }
  g_body = &body;
  g_grid_dim = grid;
  g_block_dim = block;
  g_blk.nthreads = (int)nthreads;
  for (int64_t b = 0; b < total; ++b) {
    if (!sampled(b, total)) continue;
    g_block_idx = Dim{(unsigned)(b % grid.x), (unsigned)((b / grid.x) % grid.y), (unsigned)(b / ((int64_t)grid.x * grid.y))};
    run_block();
  }
  if (g_dyn_lds) {
    __asan_unpoison_memory_region(g_dyn_lds, lds_alloc.map_size - 2 * kGuard);
    munmap(lds_alloc.map, lds_alloc.map_size);
  }
  g_dyn_lds = nullptr;
  g_body = nullptr;
}

}  // namespace emu

// ---- control interface for the Python test driver ----
extern "C" {

__attribute__((visibility("default"))) void* emu_alloc(size_t n) {
  emu::Alloc a{};
  void* p = emu::guarded_map(n, a);
  if (!p) return nullptr;
  emu::g_allocs[a.base] = a;
  return p;
}

__attribute__((visibility("default"))) int emu_free(void* p) {
  auto it = emu::g_allocs.find(reinterpret_cast<uintptr_t>(p));
  if (it == emu::g_allocs.end()) return 1;
  emu::Alloc a = it->second;
  emu::g_allocs.erase(it);
  if (a.map) {
    __asan_unpoison_memory_region(reinterpret_cast<void*>(a.base), a.map_size - 2 * emu::kGuard);
    munmap(a.map, a.map_size);
  }
  return 0;
}

// registers memory the driver did not get from emu_alloc (buffer-resource checks only)
__attribute__((visibility("default"))) void emu_register(const void* p, size_t n) {
  emu::Alloc a{reinterpret_cast<uintptr_t>(p), n, nullptr, 0};
  emu::g_allocs[a.base] = a;
}

__attribute__((visibility("default"))) void emu_set_sample(int64_t head, int64_t tail, int64_t stride) {
  emu::g_sample_head = head;
  emu::g_sample_tail = tail;
  emu::g_sample_stride = stride;
}

__attribute__((visibility("default"))) void emu_set_lds_dma_mode(int mode) { emu::g_lds_dma_mode = mode; }

__attribute__((visibility("default"))) void emu_set_log(int on) {
  emu::g_log = on != 0;
  emu::g_log_text.clear();
}

__attribute__((visibility("default"))) const char* emu_log_text(void) { return emu::g_log_text.c_str(); }

__attribute__((visibility("default"))) void emu_stats(int64_t* out) {
  for (int i = 0; i < emu::kNStats; ++i) out[i] = emu::g_stats[i];
}

__attribute__((visibility("default"))) void emu_reset_stats(void) {
  for (auto& s : emu::g_stats) s = 0;
}

}  // extern "C"
