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

// ---- cross-lane moves without the LDS crossbar -------------------------------
// DPP (data-parallel primitives) read a neighbour lane's VGPR inside the VALU:
// quad_perm within 4 lanes, row_ror within 16-lane rows.  row_ror:n makes lane
// i read lane (i - n) mod 16 of its row.  ds_bpermute (what __shfl_xor lowers
// to) goes through the LDS crossbar and costs ~100+ cycles of latency per use.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, x)));
}
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kRowRor4 = 0x124, kRowRor8 = 0x128, kRowRor12 = 0x12C;

// Value of lane (lane ^ M).  M <= 8 stays inside a 16-lane row (DPP); 16 and
// 32 use the gfx950 lane swaps (VALU, no LDS crossbar): with both operands x,
// v_permlane16_swap returns (x with odd rows replaced by the even rows below,
// x with even rows replaced by the odd rows above), v_permlane32_swap the same
// for the two 32-lane halves.
template <int M>
__device__ __forceinline__ float lane_xor(float x) {
  if constexpr (M == 1) {
    return dpp_f<kQuadXor1>(x);
  } else if constexpr (M == 2) {
    return dpp_f<kQuadXor2>(x);
  } else if constexpr (M == 4) {
    const float from_lo = dpp_f<kRowRor4>(x);   // lane i - 4
    const float from_hi = dpp_f<kRowRor12>(x);  // lane i + 4
    return (threadIdx.x & 4) ? from_lo : from_hi;
  } else if constexpr (M == 8) {
    return dpp_f<kRowRor8>(x);
  } else if constexpr (M == 16 || M == 32) {
    const int i = __builtin_bit_cast(int, x);
    const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(i, i, false, false)
                           : __builtin_amdgcn_permlane32_swap(i, i, false, false);
    return __builtin_bit_cast(float, (int)((threadIdx.x & M) ? r[0] : r[1]));
  } else {
    return __shfl_xor(x, M, 64);
  }
}

// All-reduce inside each 16-lane row (every lane gets its row's result).
// Sum / max are order-free here (integers, or max), so any pairing is exact.
__device__ __forceinline__ int row16_sum_int(int v) {
  v += dpp_i<kQuadXor1>(v);
  v += dpp_i<kQuadXor2>(v);
  v += dpp_i<kRowRor4>(v);
  v += dpp_i<kRowRor8>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kQuadXor1>(v));
  v = fmaxf(v, dpp_f<kQuadXor2>(v));
  v = fmaxf(v, dpp_f<kRowRor4>(v));
  v = fmaxf(v, dpp_f<kRowRor8>(v));
  return v;
}
// Whole-wave results, uniform across the wave: row reduction, then the four
// row results read into scalars.
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  const int i = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ int wave_sum_int(int v) {
  v = row16_sum_int(v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}
// Sum over each 32-lane half of the wave (lanes 0-31 and 32-63), uniform per half.
__device__ __forceinline__ int half_sum_int(int v) {
  v = row16_sum_int(v);
  const int lo = __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16);
  const int hi = __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
  return (threadIdx.x & 32) ? hi : lo;
}

}  // namespace ifrd
