// Device-side helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

namespace ifrd {

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// fp32 -> fp16 round-to-nearest-even of an fp32 VALUE.  The empty asm pins
// the operand in a VGPR as a finished fp32 result: otherwise the compiler may
// fold the producing multiply/add into a mixed-precision instruction that
// rounds the exact result straight to fp16 (one rounding instead of the
// contract's fp32-then-fp16), which differs in rare ulp cases.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float fp16r(float f) {
  asm volatile("" : "+v"(f));
  return (float)(_Float16)f;
}

// Half-away-from-zero after clamping to +-127: trunc(v + copysign(0.5, v)),
// the reference trunk rounding (dashq.cpp:243-246).
__device__ __forceinline__ int quant_half_away(float x, float inv) {
  float v = x * inv;
  v = fminf(fmaxf(v, -127.0f), 127.0f);
  return (int)__builtin_truncf(v + __builtin_copysignf(0.5f, v));
}
// Round-to-nearest-even after the clamp (the reference lm_head rounding).
__device__ __forceinline__ int quant_rne(float x, float inv) {
  float v = x * inv;
  v = fminf(fmaxf(v, -127.0f), 127.0f);
  return (int)__builtin_rintf(v);
}

// Order LDS traffic between lanes of one wave (no s_barrier needed).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace ifrd
