// CPU emulation runtime for tests/hipemu/hip/hip_runtime.h (test
// infrastructure only).  One OS thread runs the blocks of a launch one after
// another; inside a block every GPU thread is a fiber with its own stack.
// Fibers switch only at exchange points (cross-lane operations, barriers) and
// at exit, so a wavefront behaves as if its lanes ran in lockstep.
#include <hip/hip_runtime.h>

#include <sys/mman.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#ifdef EMU_ASAN
#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#endif

extern "C" void emu_swap(void** save_sp, void* new_sp);
asm(R"(
.text
.globl emu_swap
.type emu_swap,@function
emu_swap:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
.size emu_swap,.-emu_swap
)");

namespace emu {
namespace {

constexpr size_t kStack = 512 * 1024;
constexpr int kMaxThreads = 1024;

enum State { RUNNABLE, WAIT_WAVE, WAIT_BLOCK, DONE };

struct Fiber {
  ThreadCtx ctx;
  void* sp = nullptr;
  char* stack = nullptr;
  State st = DONE;
  unsigned wait_gen = 0;
  int slot_sel = 0;  // exchange buffer this lane reads next
};

struct Wave {
  uint64_t live_mask = 0;
  int live = 0, arrived = 0;
  unsigned gen = 0;
  int op = 0;
  int buf = 0;  // buffer being filled
  unsigned char slots[2][64 * 64];
};

struct Block {
  int live = 0, arrived = 0;
  unsigned gen = 0;
};

struct Sched {
  Fiber fibers[kMaxThreads];
  Wave waves[kMaxThreads / 64];
  Block block;
  int nthreads = 0;
  int current = -1;
  void* main_sp = nullptr;
  KernelBody body = nullptr;
  void* args = nullptr;
  std::vector<unsigned char> dyn;
  size_t dyn_bytes = 0;
  bool failed = false;
  std::string why;
#ifdef EMU_ASAN
  void* main_fake = nullptr;
  const void* main_bottom = nullptr;
  size_t main_size = 0;
#endif
};

Sched* g_s = nullptr;
int g_err = hipSuccess;
thread_local ThreadCtx g_host_ctx{};

Sched& S() {
  if (!g_s) {
    g_s = new Sched();
    for (int i = 0; i < kMaxThreads; ++i) {
      void* m = mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE,
                     -1, 0);
      if (m == MAP_FAILED) {
        std::fprintf(stderr, "[hipemu] stack mmap failed\n");
        std::abort();
      }
      g_s->fibers[i].stack = static_cast<char*>(m);
    }
  }
  return *g_s;
}

void fail(const std::string& why) {
  Sched& s = S();
  if (!s.failed) {
    s.failed = true;
    s.why = why;
  }
  std::fprintf(stderr, "[hipemu] ERROR: %s\n", why.c_str());
  std::fflush(stderr);
  std::abort();
}

// Switch from the current fiber to the scheduler (main context).
void to_main() {
  Sched& s = S();
  Fiber& f = s.fibers[s.current];
#ifdef EMU_ASAN
  void* fake = nullptr;
  __sanitizer_start_switch_fiber(f.st == DONE ? nullptr : &fake, s.main_bottom, s.main_size);
#endif
  emu_swap(&f.sp, s.main_sp);
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
}

[[noreturn]] void fiber_entry() {
  Sched& s = S();
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(nullptr, &s.main_bottom, &s.main_size);
#endif
  s.body(s.args);
  Fiber& f = s.fibers[s.current];
  f.st = DONE;
  Wave& w = s.waves[f.ctx.wave];
  w.live -= 1;
  w.live_mask &= ~(uint64_t(1) << f.ctx.lane);
  s.block.live -= 1;
  // a pending rendezvous may now be complete without this lane
  if (w.arrived > 0 && w.arrived >= w.live) {
    w.arrived = 0;
    w.buf ^= 1;
    w.gen++;
  }
  if (s.block.arrived > 0 && s.block.arrived >= s.block.live) {
    s.block.arrived = 0;
    s.block.gen++;
  }
  to_main();
  std::abort();
}

void start_fiber(Fiber& f) {
#ifdef EMU_ASAN
  // a reused stack still carries the redzone poison of earlier frames
  __asan_unpoison_memory_region(f.stack, kStack);
#endif
  char* top = f.stack + kStack;
  top = reinterpret_cast<char*>(reinterpret_cast<uintptr_t>(top) & ~uintptr_t(15));
  void** sp = reinterpret_cast<void**>(top);
  *--sp = nullptr;                                    // fake return address of fiber_entry
  *--sp = reinterpret_cast<void*>(&fiber_entry);      // popped by ret
  for (int i = 0; i < 6; ++i) *--sp = nullptr;        // rbp rbx r12 r13 r14 r15
  f.sp = sp;
  f.st = RUNNABLE;
}

bool runnable(const Sched& s, const Fiber& f) {
  if (f.st == RUNNABLE) return true;
  if (f.st == WAIT_WAVE) return s.waves[f.ctx.wave].gen != f.wait_gen;
  if (f.st == WAIT_BLOCK) return s.block.gen != f.wait_gen;
  return false;
}

void run_block(Sched& s, dim3 g, dim3 b, unsigned bx, unsigned by, unsigned bz) {
  const int n = (int)(b.x * b.y * b.z);
  s.nthreads = n;
  const int nw = (n + 63) / 64;
  for (int w = 0; w < nw; ++w) {
    Wave& wv = s.waves[w];
    wv.live = std::min(64, n - 64 * w);
    wv.live_mask = wv.live == 64 ? ~uint64_t(0) : ((uint64_t(1) << wv.live) - 1);
    wv.arrived = 0;
    wv.gen = 0;
    wv.op = 0;
    wv.buf = 0;
  }
  s.block.live = n;
  s.block.arrived = 0;
  s.block.gen = 0;
  if (s.dyn_bytes) std::memset(s.dyn.data(), 0xCD, s.dyn_bytes);
  for (int t = 0; t < n; ++t) {
    Fiber& f = s.fibers[t];
    f.ctx.tid = Idx{(unsigned)(t % b.x), (unsigned)((t / b.x) % b.y), (unsigned)(t / (b.x * b.y))};
    f.ctx.bid = Idx{bx, by, bz};
    f.ctx.bdim = Idx{b.x, b.y, b.z};
    f.ctx.gdim = Idx{g.x, g.y, g.z};
    f.ctx.lane = t & 63;
    f.ctx.wave = t >> 6;
    f.slot_sel = 0;
    start_fiber(f);
  }
  int done = 0;
  int i = 0;
  while (done < n) {
    int k = 0;
    while (k < n && !runnable(s, s.fibers[(i + k) % n])) ++k;
    if (k == n) {
      char buf[256];
      std::snprintf(buf, sizeof buf, "deadlock in block (%u,%u,%u): no thread can proceed", bx, by, bz);
      fail(buf);
    }
    i = (i + k) % n;
    Fiber& f = s.fibers[i];
    f.st = RUNNABLE;
    s.current = i;
#ifdef EMU_ASAN
    void* fake = nullptr;
    __sanitizer_start_switch_fiber(&fake, f.stack, kStack);
#endif
    emu_swap(&s.main_sp, f.sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
    if (f.st == DONE) ++done;
    i = (i + 1) % n;
  }
  s.current = -1;
}

}  // namespace

ThreadCtx* cur() {
  Sched& s = S();
  if (s.current < 0) return &g_host_ctx;
  return &s.fibers[s.current].ctx;
}

void* dyn_shared() { return S().dyn.data(); }

uint64_t live_mask_of_current_wave() {
  Sched& s = S();
  return s.waves[s.fibers[s.current].ctx.wave].live_mask;
}

void emu_set_err(int e) {
  if (e != hipSuccess) g_err = e;
}

const unsigned char* wave_exchange(const void* mine, int bytes, int op) {
  Sched& s = S();
  if (s.current < 0) fail("cross-lane operation outside a kernel");
  Fiber& f = s.fibers[s.current];
  Wave& w = s.waves[f.ctx.wave];
  if (bytes > 64) fail("exchange payload > 64 bytes");
  if (w.arrived == 0) {
    w.op = op;
  } else if (w.op != op) {
    char b[160];
    std::snprintf(b, sizeof b, "divergent cross-lane operations in wave %d (op %d vs %d)", f.ctx.wave, w.op, op);
    fail(b);
  }
  const int buf = w.buf;
  std::memcpy(&w.slots[buf][(size_t)f.ctx.lane * 64], mine, (size_t)bytes);
  w.arrived++;
  if (w.arrived >= w.live) {
    w.arrived = 0;
    w.buf ^= 1;
    w.gen++;
  } else {
    f.st = WAIT_WAVE;
    f.wait_gen = w.gen;
    to_main();
  }
  return w.slots[buf];
}

void wave_barrier() {
  int z = 0;
  (void)wave_exchange(&z, 4, 100);
}

void block_barrier() {
  Sched& s = S();
  if (s.current < 0) fail("__syncthreads outside a kernel");
  Fiber& f = s.fibers[s.current];
  Wave& w = s.waves[f.ctx.wave];
  if (w.arrived != 0) fail("__syncthreads while the wave is inside a cross-lane operation");
  s.block.arrived++;
  if (s.block.arrived >= s.block.live) {
    s.block.arrived = 0;
    s.block.gen++;
  } else {
    f.st = WAIT_BLOCK;
    f.wait_gen = s.block.gen;
    to_main();
  }
}

int launch_raw(KernelBody body, void* args, dim3 g, dim3 b, size_t shmem) {
  Sched& s = S();
  const long n = (long)b.x * b.y * b.z;
  if (n <= 0 || n > kMaxThreads || g.x == 0 || g.y == 0 || g.z == 0 || g.y > 65535 || g.z > 65535 ||
      shmem > 160 * 1024) {
    std::fprintf(stderr, "[hipemu] invalid launch: grid (%u,%u,%u) block (%u,%u,%u) shmem %zu\n", g.x, g.y,
                 g.z, b.x, b.y, b.z, shmem);
    return hipErrorInvalidValue;
  }
  if (s.current >= 0) fail("kernel launch from inside a kernel");
  s.body = body;
  s.args = args;
  s.dyn_bytes = shmem;
  s.dyn.assign(shmem ? shmem : 1, 0);
  for (unsigned bz = 0; bz < g.z; ++bz)
    for (unsigned by = 0; by < g.y; ++by)
      for (unsigned bx = 0; bx < g.x; ++bx) run_block(s, g, b, bx, by, bz);
  // the dynamic LDS of this launch is released (ASan sees any later use)
  std::vector<unsigned char>().swap(s.dyn);
  return hipSuccess;
}

}  // namespace emu

// ---- builtins ------------------------------------------------------------------------

void emu_global_load_lds(const void* g, void* l, unsigned size, int offset, int aux) {
  if (offset != 0 || aux != 0 || (size != 1 && size != 2 && size != 4 && size != 12 && size != 16))
    emu::fail("global_load_lds: offset, aux or size not emulated");
  const uint64_t live = emu::live_mask_of_current_wave();
  const unsigned char* s = emu::wave_exchange(&l, sizeof(void*), emu::kOpFirst);
  for (int k = 0; k < 64; ++k)
    if (((live >> k) & 1) && emu::lane_value<void*>(s, k) != l) emu::fail("global_load_lds: LDS address not wave-uniform");
  std::memcpy(static_cast<unsigned char*>(l) + (size_t)emu::cur()->lane * size, g, size);
}

int emu_readfirstlane(int v) {
  const uint64_t live = emu::live_mask_of_current_wave();
  const unsigned char* s = emu::wave_exchange(&v, 4, emu::kOpFirst);
  return emu::lane_value<int>(s, __builtin_ctzll(live));
}

int emu_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  const unsigned char* s = emu::wave_exchange(&src, 4, emu::kOpDpp);
  const int l = emu::cur()->lane;
  if (row_mask != 0xF || bank_mask != 0xF) {
    std::fprintf(stderr, "[hipemu] DPP row/bank masks other than 0xF are not emulated\n");
    std::abort();
  }
  int from = -1;
  if (ctrl >= 0 && ctrl <= 0xFF) {  // quad_perm
    from = (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
  } else if (ctrl >= 0x101 && ctrl <= 0x10F) {  // row_shl
    const int n = ctrl & 0xF, r = l & 15;
    from = r + n < 16 ? l + n : -1;
  } else if (ctrl >= 0x111 && ctrl <= 0x11F) {  // row_shr
    const int n = ctrl & 0xF, r = l & 15;
    from = r - n >= 0 ? l - n : -1;
  } else if (ctrl >= 0x121 && ctrl <= 0x12F) {  // row_ror: lane i reads lane (i - n) mod 16
    const int n = ctrl & 0xF;
    from = (l & ~15) + (((l & 15) - n + 16) & 15);
  } else {
    std::fprintf(stderr, "[hipemu] DPP control 0x%x is not emulated\n", ctrl);
    std::abort();
  }
  if (from < 0) return bound_ctrl ? 0 : old;
  return emu::lane_value<int>(s, from);
}

// v_permlane16_swap / v_permlane32_swap (CDNA4 ISA): the odd 16-lane rows
// (upper 32-lane half) of the first operand trade places with the even rows
// (lower half) of the second; returns (new first, new second).
static emu_v2u permlane_swap(unsigned vdst, unsigned vsrc, int span) {
  const unsigned pair[2] = {vdst, vsrc};
  const unsigned char* s = emu::wave_exchange(pair, 8, emu::kOpShfl);
  const int l = emu::cur()->lane;
  auto at = [&](int lane, int k) { return emu::lane_value<unsigned long long>(s, lane) >> (32 * k) & 0xFFFFFFFFu; };
  emu_v2u r;
  const bool upper = (l & span) != 0;
  r[0] = upper ? (unsigned)at(l - span, 1) : (unsigned)at(l, 0);
  r[1] = upper ? (unsigned)at(l, 1) : (unsigned)at(l + span, 0);
  return r;
}
emu_v2u emu_permlane16_swap(unsigned vdst, unsigned vsrc, bool, bool) { return permlane_swap(vdst, vsrc, 16); }
emu_v2u emu_permlane32_swap(unsigned vdst, unsigned vsrc, bool, bool) { return permlane_swap(vdst, vsrc, 32); }

emu_v4i emu_mfma_i32_16x16x64_i8(emu_v4i a, emu_v4i b, emu_v4i c) {
  struct P {
    emu_v4i a, b;
  } mine{a, b};
  const unsigned char* s = emu::wave_exchange(&mine, sizeof(P), emu::kOpMfma);
  const int l = emu::cur()->lane;
  const int n = l & 15, g = l >> 4;
  int8_t A[4][64], B[64];
  for (int kb = 0; kb < 4; ++kb) {
    for (int r = 0; r < 4; ++r) std::memcpy(&A[r][16 * kb], s + (size_t)(4 * g + r + 16 * kb) * 64, 16);
    std::memcpy(&B[16 * kb], s + (size_t)(n + 16 * kb) * 64 + 16, 16);
  }
  emu_v4i d = c;
  for (int r = 0; r < 4; ++r) {
    long acc = 0;
    for (int k = 0; k < 64; ++k) acc += (long)A[r][k] * (long)B[k];
    d[r] = (int)((long)c[r] + acc);
  }
  return d;
}

emu_v4f emu_mfma_f32_16x16x32_f16(emu_v8h a, emu_v8h b, emu_v4f c) {
  struct P {
    emu_v8h a, b;
  } mine{a, b};
  const unsigned char* s = emu::wave_exchange(&mine, sizeof(P), emu::kOpMfma);
  const int l = emu::cur()->lane;
  const int n = l & 15, g = l >> 4;
  _Float16 A[4][32], B[32];
  for (int kb = 0; kb < 4; ++kb) {
    for (int r = 0; r < 4; ++r) std::memcpy(&A[r][8 * kb], s + (size_t)(4 * g + r + 16 * kb) * 64, 16);
    std::memcpy(&B[8 * kb], s + (size_t)(n + 16 * kb) * 64 + 16, 16);
  }
  emu_v4f d = c;
  for (int r = 0; r < 4; ++r) {
    double acc = 0.0;
    for (int k = 0; k < 32; ++k) acc += (double)(float)A[r][k] * (double)(float)B[k];
    d[r] = (float)((double)c[r] + acc);
  }
  return d;
}

// ---- runtime API ------------------------------------------------------------------------
namespace {
std::map<void*, size_t>& allocs() {
  static std::map<void*, size_t> m;
  return m;
}
}  // namespace

hipError_t hipGetDeviceCount(int* n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d) {
  if (d != 0 || a != hipDeviceAttributeMultiprocessorCount) return hipErrorInvalidValue;
  *v = 256;
  return hipSuccess;
}
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int) {
  std::memset(p, 0, sizeof *p);
  std::snprintf(p->name, sizeof p->name, "hipemu");
  std::snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950:sramecc+:xnack-");
  p->totalGlobalMem = (size_t)288 << 30;
  p->multiProcessorCount = 256;
  return hipSuccess;
}
hipError_t hipMalloc(void** p, size_t n) {
  // uninitialized device memory holds a recognizable pattern (0xCD bytes)
  void* q = std::malloc(n ? n : 1);
  if (!q) return hipErrorOutOfMemory;
  std::memset(q, 0xCD, n);
  allocs()[q] = n;
  *p = q;
  return hipSuccess;
}
hipError_t hipFree(void* p) {
  if (!p) return hipSuccess;
  auto it = allocs().find(p);
  if (it == allocs().end()) {
    std::fprintf(stderr, "[hipemu] hipFree of a pointer hipMalloc did not return\n");
    std::abort();
  }
  allocs().erase(it);
  std::free(p);
  return hipSuccess;
}
hipError_t hipHostMalloc(void** p, size_t n, unsigned) { return hipMalloc(p, n); }
hipError_t hipHostFree(void* p) { return hipFree(p); }
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
  if (n) std::memmove(d, s, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t) {
  return hipMemcpy(d, s, n, k);
}
hipError_t hipMemset(void* d, int v, size_t n) {
  if (n) std::memset(d, v, n);
  return hipSuccess;
}
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t) { return hipMemset(d, v, n); }
hipError_t hipStreamCreate(hipStream_t* s) {
  *s = reinterpret_cast<hipStream_t>(new int(1));
  return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) { return hipStreamCreate(s); }
hipError_t hipStreamDestroy(hipStream_t s) {
  delete reinterpret_cast<int*>(s);
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t* e) {
  *e = reinterpret_cast<hipEvent_t>(new double(0.0));
  return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { return hipEventCreate(e); }
// launches run synchronously in the emulation, so stream order is program order
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t e) {
  delete reinterpret_cast<double*>(e);
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
  *reinterpret_cast<double*>(e) =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
  *ms = (float)(*reinterpret_cast<double*>(b) - *reinterpret_cast<double*>(a));
  return hipSuccess;
}
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int v) {
  return v <= 160 * 1024 ? hipSuccess : hipErrorInvalidValue;
}
hipError_t hipGetLastError() {
  const int e = emu::g_err;
  emu::g_err = hipSuccess;
  return e;
}
hipError_t hipPeekAtLastError() { return emu::g_err; }
const char* hipGetErrorString(hipError_t e) {
  switch (e) {
    case hipSuccess: return "hipSuccess";
    case hipErrorInvalidValue: return "hipErrorInvalidValue";
    case hipErrorOutOfMemory: return "hipErrorOutOfMemory";
    default: return "hip error";
  }
}
