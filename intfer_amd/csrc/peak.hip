// Measured peaks of one MI355X: the denominators reported next to the nominal
// ones (8 TB/s HBM, 5 POP/s int8 and 2.5 PFLOP/s fp16 dense MFMA).
//   peak_read_kernel   a streaming read of a buffer far above the 256 MB
//                      Infinity Cache: every 16-byte word once, nontemporal
//   peak_mfma_kernel   back-to-back independent v_mfma_i32_16x16x64_i8 (or
//                      v_mfma_f32_16x16x32_f16) in two waves per SIMD
// Results are folded into one word per thread so nothing is dead code.
#include <hip/hip_runtime.h>

#include "ifr_dev.h"
#include "intfer_amd.h"

namespace ifrh {
int fail(int code, const char* fmt, ...);
}

namespace {

constexpr int kReadBlocks = 4096, kReadThreads = 256;

__global__ __launch_bounds__(kReadThreads) void peak_read_kernel(const v4i* __restrict__ src, size_t n16,
                                                                 uint32_t* out) {
  const size_t stride = (size_t)gridDim.x * kReadThreads;
  size_t i = (size_t)blockIdx.x * kReadThreads + threadIdx.x;
  uint32_t acc = 0;
  // four loads in flight per thread, then the remainder
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4i a = __builtin_nontemporal_load(src + i);
    const v4i b = __builtin_nontemporal_load(src + i + stride);
    const v4i c = __builtin_nontemporal_load(src + i + 2 * stride);
    const v4i d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= (uint32_t)(a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n16; i += stride) {
    const v4i a = __builtin_nontemporal_load(src + i);
    acc ^= (uint32_t)(a.x ^ a.y ^ a.z ^ a.w);
  }
  out[(size_t)blockIdx.x * kReadThreads + threadIdx.x] = acc;
}

// 8 independent accumulators per wave, `iters` rounds of 8 MFMAs.
template <bool F16>
__global__ __launch_bounds__(256) void peak_mfma_kernel(int iters, uint32_t seed, uint32_t* out) {
  const uint32_t t = threadIdx.x + seed;
  if constexpr (!F16) {
    const v4i a = {(int)(t * 0x01010101u), (int)(t * 0x02030405u), (int)(t ^ 0x5A5A5A5Au), (int)(t + 7)};
    const v4i b = {(int)(t * 0x0F0E0D0Cu), (int)(t ^ 0x33333333u), (int)(t * 3u), (int)(t + 11)};
    v4i acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = (v4i){j, 0, 0, 0};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[j].x + acc[j].y + acc[j].z + acc[j].w;
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = (uint32_t)s;
  } else {
    v8h a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (_Float16)((float)((t + e) & 7) * 0.125f);
      b[e] = (_Float16)((float)((t * 3 + e) & 7) * 0.0625f);
    }
    v4f acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = (v4f){(float)j, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[j].x + acc[j].y + acc[j].z + acc[j].w;
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = __float_as_uint(s);
  }
}

// HIP-event milliseconds of `reps` launches of f on the stream.
template <typename F>
int timed(hipStream_t st, int reps, F f, double* ms) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return ifrh::fail(IFR_EDEVICE, "hipEventCreate");
  if (hipEventCreate(&b) != hipSuccess) {
    hipEventDestroy(a);
    return ifrh::fail(IFR_EDEVICE, "hipEventCreate");
  }
  f();  // untimed first launch
  hipEventRecord(a, st);
  for (int r = 0; r < reps; ++r) f();
  hipEventRecord(b, st);
  hipError_t e = hipEventSynchronize(b);
  float t = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
  if (e == hipSuccess) e = hipGetLastError();
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (e != hipSuccess) return ifrh::fail(IFR_EDEVICE, "peak kernel: %s", hipGetErrorString(e));
  *ms = t;
  return IFR_OK;
}

}  // namespace

extern "C" {

int ifr_peak_read(ifr_ctx* c, const void* buf_d, size_t bytes, int32_t reps, double* gbps) {
  if (!c || !buf_d || !gbps || reps <= 0) return ifrh::fail(IFR_EINVAL, "peak read: null arg or reps <= 0");
  if (bytes < ((size_t)1 << 30) || bytes % 16) return ifrh::fail(IFR_EINVAL, "peak read: %zu bytes (>= 1 GiB, x16)", bytes);
  hipStream_t st = static_cast<hipStream_t>(ifr_ctx_stream(c));
  uint32_t* out = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&out), (size_t)kReadBlocks * kReadThreads * 4) != hipSuccess)
    return ifrh::fail(IFR_ENOMEM, "peak read: scratch");
  double ms = 0;
  const int r = timed(st, reps, [&] {
    hipLaunchKernelGGL(peak_read_kernel, dim3(kReadBlocks), dim3(kReadThreads), 0, st,
                       static_cast<const v4i*>(buf_d), bytes / 16, out);
  }, &ms);
  hipStreamSynchronize(st);
  hipFree(out);
  if (r) return r;
  *gbps = (double)bytes * reps / (ms * 1e-3) / 1e9;
  return IFR_OK;
}

int ifr_peak_mfma(ifr_ctx* c, int32_t dtype, int32_t iters, int32_t reps, double* tops) {
  if (!c || !tops || reps <= 0 || iters <= 0 || (dtype != 0 && dtype != 1))
    return ifrh::fail(IFR_EINVAL, "peak mfma: dtype %d, iters %d, reps %d", dtype, iters, reps);
  hipStream_t st = static_cast<hipStream_t>(ifr_ctx_stream(c));
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
    return ifrh::fail(IFR_EDEVICE, "peak mfma: CU count");
  const int blocks = 2 * ncu;  // 8 waves per CU: two per SIMD
  uint32_t* out = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&out), (size_t)blocks * 256 * 4) != hipSuccess)
    return ifrh::fail(IFR_ENOMEM, "peak mfma: scratch");
  double ms = 0;
  const int r = timed(st, reps, [&] {
    if (dtype == 0) hipLaunchKernelGGL(peak_mfma_kernel<false>, dim3(blocks), dim3(256), 0, st, iters, 1u, out);
    else hipLaunchKernelGGL(peak_mfma_kernel<true>, dim3(blocks), dim3(256), 0, st, iters, 1u, out);
  }, &ms);
  hipStreamSynchronize(st);
  hipFree(out);
  if (r) return r;
  // per MFMA: 16 x 16 outputs x K (64 int8 or 32 fp16) multiply-adds, 2 ops each
  const double per = 2.0 * 16 * 16 * (dtype == 0 ? 64 : 32);
  const double ops = per * 8.0 * iters * (blocks * 4.0) * reps;
  *tops = ops / (ms * 1e-3) / 1e12;
  return IFR_OK;
}

}  // extern "C"
