// W2A8 / W4A8 / W8A8 GEMM with grouped activation scales: the reference's
// DPAS fold (dpas48_tiled, src/gemm/quant_gemm.cpp:3492-3791; the per-op math
// :3602-3736, activation group GA :3502, As[r][k0 / GA] :3614).  For each
// 32-wide K op in ascending order (k0 = 32 o):
//
//   T = sum a_q(m,k) c(n,k),  S = sum a_q(m,k)          exact int32 over the op
//   acc += as(m, k0/GA) * ws(n, k0/128) * alpha * (2T - C S) * (1/C)
//   out(m,n) = fp16_rne(acc)
//
// in the source's left-to-right order, every product and the add rounded
// (the build compiles with -ffp-contract=off).  2T - C S is an integer below
// 2^24, exact in fp32.  Codebook linears only: the fold has no zero term.
//
// A parity operating point beside the per-group fold of qgemm.hip (the
// engine's contract): one wave per 16 x 16 output tile over the whole K.
// The op is half of one int8 MFMA K step (64 columns): lanes 0-31 of the A
// operand hold its first 32 columns, lanes 32-63 the second, so masking the
// other half gives T per op, and the same masked A against a B of ones gives
// S per op and row in the layout of T.
#include "ifr_dev.h"
#include "ifr_kernels.h"

namespace ifrk {
namespace {

// Plain codes of one lane for one K step as the int8 B operand: dword d
// holds codes 4d .. 4d + 3 in bytes 0..3 (INT8 stored as c - 128).
template <int BITS>
__device__ __forceinline__ v4i ga_codes(const uint32_t (&src)[BITS / 2]) {
  v4i r;
  if constexpr (BITS == 2) {
    const uint32_t w = src[0];
    r.x = (int)(w & 0x03030303u);
    r.y = (int)((w >> 2) & 0x03030303u);
    r.z = (int)((w >> 4) & 0x03030303u);
    r.w = (int)((w >> 6) & 0x03030303u);
  } else if constexpr (BITS == 4) {
    const uint32_t w0 = src[0], w1 = src[1];
    r.x = (int)(w0 & 0x0F0F0F0Fu);
    r.y = (int)((w0 >> 4) & 0x0F0F0F0Fu);
    r.z = (int)(w1 & 0x0F0F0F0Fu);
    r.w = (int)((w1 >> 4) & 0x0F0F0F0Fu);
  } else {
    r.x = (int)src[0];
    r.y = (int)src[1];
    r.z = (int)src[2];
    r.w = (int)src[3];
  }
  return r;
}

template <int BITS>
__global__ __launch_bounds__(256) void qgemm_ga_kernel(GaArgs p) {
  constexpr float C = (float)((1 << BITS) - 1);
  constexpr float Cinv = 1.0f / C;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // column tile
  if (t >= p.N / 16) return;  // (no barrier in this kernel)
  const int rb = blockIdx.y;  // 16-row block
  const int c = lane & 15, q = lane >> 4;
  const int nsl = p.K / p.ga;
  // result register r of lane (c, q) holds row 4q + r of the block, column c
  int rows[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) rows[r] = min(16 * rb + 4 * q + r, p.M - 1);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const v4i zero = {0, 0, 0, 0};
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  const int8_t* abase = p.a + (size_t)rb * p.nsteps * 1024 + 16 * lane;
  const uint32_t* cbase = p.codes + (size_t)t * p.nsteps * 64 * (BITS / 2) + lane * (BITS / 2);
  // R K steps of operands in flight: slot d of the ring holds step s0 + d and
  // is refilled with step s0 + d + R (clamped to the last step, in bounds)
  // as soon as its step is computed
  constexpr int R = 8;
  // (both ops of a step share one activation slice, ga being a multiple of
  // 64, and one 128-wide weight group)
  struct StepOps {
    v4i A;
    uint32_t w[BITS / 2];
    float as[4];
    uint32_t sz;
  } ring[R];
  auto load = [&](StepOps& o, int s) {
    s = min(s, p.nsteps - 1);
    o.A = *reinterpret_cast<const v4i*>(abase + (size_t)s * 1024);
    const uint32_t* src = cbase + (size_t)s * 64 * (BITS / 2);
#pragma unroll
    for (int i = 0; i < BITS / 2; ++i) o.w[i] = src[i];
#pragma unroll
    for (int r = 0; r < 4; ++r) o.as[r] = p.as[(size_t)rows[r] * nsl + 64 * s / p.ga];
    o.sz = p.sz[((size_t)t * p.ng + s / 2) * 16 + c];
  };
#pragma unroll
  for (int d = 0; d < R; ++d) load(ring[d], d);
  for (int s0 = 0; s0 < p.nsteps; s0 += R)
#pragma unroll
  for (int d = 0; d < R; ++d) {
    const int s = s0 + d;
    if (s >= p.nsteps) break;
    const v4i A = ring[d].A;
    const v4i B = ga_codes<BITS>(ring[d].w);
    float asv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) asv[r] = ring[d].as[r];
    const float ws = ifrd::h2f((uint16_t)(ring[d].sz & 0xFFFFu));
    load(ring[d], s + R);
    // lanes 0-31 carry columns 64 s .. + 31 (op 2 s), lanes 32-63 the rest
    const v4i A0 = q < 2 ? A : zero, A1 = q < 2 ? zero : A;
    v4i T[2], S[2];
    T[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B, zero, 0, 0, 0);
    T[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B, zero, 0, 0, 0);
    S[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, ones, zero, 0, 0, 0);
    S[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, ones, zero, 0, 0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int32_t Tv = T[h][r];
        const int32_t Sv = S[h][r];
        if constexpr (BITS == 8) Tv += 128 * Sv;  // codes stored as c - 128
        const float dv = 2.0f * (float)Tv - C * (float)Sv;
        float x = asv[r] * ws;
        x = x * p.alpha;
        x = x * dv;
        x = x * Cinv;
        acc[r] = acc[r] + x;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 16 * rb + 4 * q + r;
    if (row < p.M) p.out[(size_t)row * p.N + 16 * t + c] = ifrd::f2h(acc[r]);
  }
}

}  // namespace

hipError_t launch_qgemm_ga(const GaArgs& p, hipStream_t st) {
  if (p.M <= 0) return hipSuccess;
  if (!p.a || !p.as || !p.codes || !p.sz || !p.out || p.N <= 0 || p.N % 16 != 0 || p.K <= 0 ||
      p.K % 128 != 0 || p.ng != p.K / 128 || p.nsteps != p.K / 64 || p.ga <= 0 || p.ga % 64 != 0 ||
      p.K % p.ga != 0 || (p.M + 15) / 16 > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((p.N / 16 + 3) / 4, (p.M + 15) / 16), block(256);
  switch (p.bits) {
    case 2: hipLaunchKernelGGL(qgemm_ga_kernel<2>, grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL(qgemm_ga_kernel<4>, grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL(qgemm_ga_kernel<8>, grid, block, 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ifrk
