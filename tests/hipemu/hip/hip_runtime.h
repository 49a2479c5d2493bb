// CPU emulation of the HIP runtime and the gfx950 device builtins used by
// intfer_amd/csrc (test infrastructure only; never part of the product).
//
// The library sources are compiled for the host against this header (it
// shadows <hip/hip_runtime.h> on the include path) and instrumented with
// AddressSanitizer, so every global, LDS and stack access of every kernel is
// bounds-checked on the CPU.  Each GPU thread runs as a fiber; lanes of a
// wavefront meet at every cross-lane operation (shuffles, DPP, readlane,
// MFMA, wave barriers) and all threads of a block at __syncthreads, which
// gives the lockstep semantics those operations need.  A block that cannot
// make progress (mismatched barriers) is reported as a deadlock.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <tuple>
#include <utility>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __restrict__ __restrict
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))

typedef int hipError_t;
enum {
  hipSuccess = 0,
  hipErrorInvalidValue = 1,
  hipErrorOutOfMemory = 2,
  hipErrorLaunchFailure = 719,
};
typedef void* hipStream_t;
typedef void* hipEvent_t;
enum hipMemcpyKind {
  hipMemcpyHostToHost = 0,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipMemcpyDeviceToDevice = 3,
  hipMemcpyDefault = 4
};
enum { hipStreamDefault = 0, hipStreamNonBlocking = 1 };
enum { hipHostMallocDefault = 0 };
enum { hipEventDefault = 0, hipEventDisableTiming = 2 };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };

struct hipDeviceProp_t {
  char name[256];
  char gcnArchName[256];
  size_t totalGlobalMem;
  int multiProcessorCount;
};

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

struct __attribute__((aligned(16))) uint4 { unsigned x, y, z, w; };
struct __attribute__((aligned(8))) uint2 { unsigned x, y; };
struct __attribute__((aligned(16))) float4 { float x, y, z, w; };
struct __attribute__((aligned(8))) float2 { float x, y; };
struct __attribute__((aligned(16))) int4 { int x, y, z, w; };
inline uint2 make_uint2(unsigned a, unsigned b) { return uint2{a, b}; }
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return uint4{a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }

inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }

namespace emu {

struct Idx {
  unsigned x, y, z;
};
struct ThreadCtx {
  Idx tid, bid, bdim, gdim;
  int lane, wave;
};
ThreadCtx* cur();
void* dyn_shared();
uint64_t live_mask_of_current_wave();

// ---- lockstep exchange points ------------------------------------------------
// Every lane of the calling wave deposits `bytes` bytes; after all live lanes
// arrived, returns a pointer to the 64 deposits (slot l = lane l), valid until
// the lane's next exchange.  `op` names the call site kind (divergence check).
const unsigned char* wave_exchange(const void* mine, int bytes, int op);
void block_barrier();
void wave_barrier();

template <typename T>
inline T lane_value(const unsigned char* slots, int l) {
  T v;
  std::memcpy(&v, slots + (size_t)l * 64, sizeof(T));
  return v;
}

typedef void (*KernelBody)(void*);
int launch_raw(KernelBody body, void* args, dim3 g, dim3 b, size_t shmem);

template <typename... P>
struct LaunchPack {
  void (*k)(P...);
  std::tuple<P...> args;
  static void run(void* self) {
    auto* s = static_cast<LaunchPack*>(self);
    std::apply(s->k, s->args);
  }
};

template <typename... P, typename... A>
int launch(void (*k)(P...), dim3 g, dim3 b, size_t shmem, A&&... a) {
  LaunchPack<P...> pk{k, std::tuple<P...>(std::forward<A>(a)...)};
  return launch_raw(&LaunchPack<P...>::run, &pk, g, b, shmem);
}

}  // namespace emu

#define threadIdx (::emu::cur()->tid)
#define blockIdx (::emu::cur()->bid)
#define blockDim (::emu::cur()->bdim)
#define gridDim (::emu::cur()->gdim)

#define hipLaunchKernelGGL(K, G, B, S, ST, ...) ((void)(ST), ::emu::emu_set_err(::emu::launch(K, dim3(G), dim3(B), (size_t)(S), ##__VA_ARGS__)))
namespace emu {
void emu_set_err(int e);
}

inline void __syncthreads() { emu::block_barrier(); }

// ---- cross-lane builtins ---------------------------------------------------------
namespace emu {
enum { kOpShfl = 1, kOpDpp = 2, kOpReadlane = 3, kOpFirst = 4, kOpMfma = 5 };
}

template <typename T>
inline T __shfl_xor(T v, int mask, int width = 64) {
  const unsigned char* s = emu::wave_exchange(&v, sizeof(T), emu::kOpShfl);
  const int l = emu::cur()->lane;
  const int base = l & ~(width - 1);
  return emu::lane_value<T>(s, base + ((l - base) ^ mask) % width);
}
template <typename T>
inline T __shfl_up(T v, unsigned delta, int width = 64) {
  const unsigned char* s = emu::wave_exchange(&v, sizeof(T), emu::kOpShfl);
  const int l = emu::cur()->lane;
  const int base = l & ~(width - 1);
  const int src = l - (int)delta;
  return src < base ? v : emu::lane_value<T>(s, src);
}
template <typename T>
inline T __shfl(T v, int src, int width = 64) {
  const unsigned char* s = emu::wave_exchange(&v, sizeof(T), emu::kOpShfl);
  const int l = emu::cur()->lane;
  const int base = l & ~(width - 1);
  return emu::lane_value<T>(s, base + (src % width));
}

inline unsigned long long __ballot(int pred) {
  const uint64_t live = emu::live_mask_of_current_wave();
  const int v = pred != 0;
  const unsigned char* s = emu::wave_exchange(&v, 4, emu::kOpShfl);
  unsigned long long m = 0;
  for (int l = 0; l < 64; ++l)
    if (((live >> l) & 1) && emu::lane_value<int>(s, l)) m |= 1ull << l;
  return m;
}

// 1 when the predicate holds on every live lane of the wave (HIP __all)
inline int __all(int pred) { return __ballot(!pred) == 0; }

inline float __int_as_float(int x) { float f; std::memcpy(&f, &x, 4); return f; }
inline float __uint_as_float(unsigned x) { float f; std::memcpy(&f, &x, 4); return f; }
inline int __float_as_int(float f) { int x; std::memcpy(&x, &f, 4); return x; }
inline unsigned __float_as_uint(float f) { unsigned x; std::memcpy(&x, &f, 4); return x; }
// v_exp_f32 (2^x); the host's exp2f stands in for the hardware approximation
#define __builtin_amdgcn_exp2f(x) exp2f(x)

inline int emu_readlane(int v, int l) {
  const unsigned char* s = emu::wave_exchange(&v, 4, emu::kOpReadlane);
  return emu::lane_value<int>(s, l);
}
int emu_readfirstlane(int v);
int emu_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl);

#define __builtin_amdgcn_readlane(...) emu_readlane(__VA_ARGS__)
#define __builtin_amdgcn_readfirstlane(...) emu_readfirstlane(__VA_ARGS__)
#define __builtin_amdgcn_update_dpp(...) emu_update_dpp(__VA_ARGS__)
typedef unsigned int emu_v2u __attribute__((ext_vector_type(2)));
emu_v2u emu_permlane16_swap(unsigned vdst, unsigned vsrc, bool fi, bool bc);
emu_v2u emu_permlane32_swap(unsigned vdst, unsigned vsrc, bool fi, bool bc);
// v_perm_b32: result byte i = byte sel_i of the 8 bytes {s0 (4-7), s1 (0-3)};
// selector 0x0C gives 0x00, 0x0D..0x0F give 0xFF (only 0..7 are used here).
inline unsigned emu_perm(unsigned s0, unsigned s1, unsigned sel) {
  const unsigned long long cat = ((unsigned long long)s0 << 32) | s1;
  unsigned r = 0;
  for (int i = 0; i < 4; ++i) {
    const unsigned k = (sel >> (8 * i)) & 0xFF;
    unsigned byte = 0;
    if (k < 8) byte = (unsigned)(cat >> (8 * k)) & 0xFF;
    else if (k == 0x0C) byte = 0;
    else if (k >= 0x0D) byte = 0xFF;
    r |= byte << (8 * i);
  }
  return r;
}
#define __builtin_amdgcn_perm(a, b, c) emu_perm((a), (b), (c))
#define __builtin_amdgcn_permlane16_swap(...) emu_permlane16_swap(__VA_ARGS__)
#define __builtin_amdgcn_permlane32_swap(...) emu_permlane32_swap(__VA_ARGS__)
#define __builtin_amdgcn_wave_barrier() ::emu::wave_barrier()
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_amdgcn_s_barrier() __syncthreads()
// LDS DMA (global_load_lds_dword*): lane l's `size` bytes from its own
// global address land at the wave-uniform LDS address + l * size (checked
// uniform); the immediate offset is not used by the library.  The wait for
// the copies (s_waitcnt) is a no-op: the copy is complete on return.
void emu_global_load_lds(const void* g, void* l, unsigned size, int offset, int aux);
#define __builtin_amdgcn_global_load_lds(...) emu_global_load_lds(__VA_ARGS__)
#define __builtin_amdgcn_s_waitcnt(x) ((void)(x))
// plain loads on the host (x86 non-temporal vector loads demand alignment)
#define __builtin_nontemporal_load(p) (*(p))

typedef int emu_v4i __attribute__((ext_vector_type(4)));
typedef float emu_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 emu_v8h __attribute__((ext_vector_type(8)));

// MFMA operand layouts (gfx950): lane l holds row / column l % 16 and the
// K slice [kw * (l / 16), +kw) (kw = 16 int8 or 8 fp16); result register r
// of lane l is D[4 * (l / 16) + r][l % 16].
emu_v4i emu_mfma_i32_16x16x64_i8(emu_v4i a, emu_v4i b, emu_v4i c);
emu_v4f emu_mfma_f32_16x16x32_f16(emu_v8h a, emu_v8h b, emu_v4f c);
inline emu_v4i emu_mfma_i8_6(emu_v4i a, emu_v4i b, emu_v4i c, int, int, int) {
  return emu_mfma_i32_16x16x64_i8(a, b, c);
}
inline emu_v4f emu_mfma_f16_6(emu_v8h a, emu_v8h b, emu_v4f c, int, int, int) {
  return emu_mfma_f32_16x16x32_f16(a, b, c);
}
#define __builtin_amdgcn_mfma_i32_16x16x64_i8(...) emu_mfma_i8_6(__VA_ARGS__)
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(...) emu_mfma_f16_6(__VA_ARGS__)

// ---- runtime API ---------------------------------------------------------------------
hipError_t hipGetDeviceCount(int* n);
hipError_t hipSetDevice(int d);
hipError_t hipGetDevice(int* d);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d);
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount };
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d);
hipError_t hipMalloc(void** p, size_t n);
template <typename T>
inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc(reinterpret_cast<void**>(p), n); }
hipError_t hipFree(void* p);
hipError_t hipHostMalloc(void** p, size_t n, unsigned flags = 0);
template <typename T>
inline hipError_t hipHostMalloc(T** p, size_t n, unsigned flags = 0) {
  return hipHostMalloc(reinterpret_cast<void**>(p), n, flags);
}
hipError_t hipHostFree(void* p);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st = nullptr);
hipError_t hipMemset(void* d, int v, size_t n);
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st = nullptr);
hipError_t hipStreamCreate(hipStream_t* s);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipDeviceSynchronize();
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned flags);
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s = nullptr);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipFuncSetAttribute(const void* f, hipFuncAttribute a, int v);
hipError_t hipGetLastError();
hipError_t hipPeekAtLastError();
// a file-scope device array is ordinary host memory here: its address is itself
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
  *p = const_cast<void*>(sym);
  return hipSuccess;
}
const char* hipGetErrorString(hipError_t e);
