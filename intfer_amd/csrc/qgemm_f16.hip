// FP16-activation dequant GEMM: the reference's default GPU linear path
// (quant_gemm_forward_usm, src/gemm/quant_gemm.cpp:359-2153), on the device
// weight layout of this library.
//
//   out(m, n) = fp16_rne( sum_k a(m, k) * w(n, k) )     fp32, k ascending
//   w(n, k)   = (scale(n, g) * alpha) * cb(code(n, k))  g = k / 128
//   cb(c)     = the canonical codebook (2c - C) / C as an fp32 constant
//               ({-1, -1/3, 1/3, 1} for INT2; canon_value, :139-144)
//
// M == 1 follows the decode kernels (:1026-1080 for INT2, :2022-2066): the
// weight stays fp32 and every step is acc = fma(a, w, acc) (the reference's
// `acc += av * w` contracted, as its device compiler's default fp model
// does).  M > 1 follows the tiled kernel (:2069-2150): the weight tile is
// rounded to fp16 when staged, so each product a * w of two halves is exact
// in fp32 and the step is one rounded add (fma gives the same bits).
//
// This path holds no integer T; it is the reference's fp16 operating point
// beside the W2A8 path (qgemm.hip), for parity with the reference's default
// numerics.  One work-item per output with a sequential k loop, as the
// reference's kernels, so the accumulation order is the reference's.
#include "ifr_dev.h"
#include "ifr_kernels.h"

namespace ifrk {
namespace {

// Codes in the fragment-major layout (pack_linear_host): column tile n / 16,
// K step k / 64, lane 16 (k % 64 / 16) + n % 16, code j = k % 16 of that
// lane in operand dword j / 4, byte j % 4 (INT8 stored as c ^ 0x80).

template <int BITS>
__device__ __forceinline__ float canon(int c) {
  if constexpr (BITS == 2) {
    return c == 0 ? -1.0f : c == 1 ? -1.0f / 3.0f : c == 2 ? 1.0f / 3.0f : 1.0f;
  } else {
    constexpr float C = (float)((1 << BITS) - 1);
    return (2.0f * (float)c - C) / C;
  }
}

// scale(n, g) * alpha, the reference's `s` (fp32)
__device__ __forceinline__ float group_scale(const F16Args& p, int n, int g) {
  const uint32_t zw = p.sz[((size_t)(n >> 4) * p.ng + g) * 16 + (n & 15)];
  return ifrd::h2f((uint16_t)(zw & 0xFFFFu)) * p.alpha;
}

// The operand dwords of column n at k = 16 q0 .. 16 q0 + 15 (q0 = k / 16):
// one lane's share of the fragment-major layout, and its 16 codes.
template <int BITS>
__device__ __forceinline__ void raw16(const F16Args& p, int n, int q0, uint32_t (&w)[BITS / 2]) {
  const int t = n >> 4, s = q0 >> 2, l = 16 * (q0 & 3) + (n & 15);
  const uint32_t* src = p.codes + (((size_t)t * p.nsteps + s) * 64 + l) * (BITS / 2);
#pragma unroll
  for (int i = 0; i < BITS / 2; ++i) w[i] = src[i];
}
template <int BITS>
__device__ __forceinline__ void decode16(const uint32_t (&w)[BITS / 2], int (&c)[16]) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int d = j >> 2, b = j & 3;
    if constexpr (BITS == 2) c[j] = (int)((w[0] >> (8 * b + 2 * d)) & 3u);
    else if constexpr (BITS == 4) c[j] = (int)((w[d >> 1] >> (8 * b + 4 * (d & 1))) & 15u);
    else c[j] = (int)(((w[d] >> (8 * b)) & 0xFFu) ^ 0x80u);
  }
}
template <int BITS>
__device__ __forceinline__ void codes16(const F16Args& p, int n, int q0, int (&c)[16]) {
  uint32_t w[BITS / 2];
  raw16<BITS>(p, n, q0, w);
  decode16<BITS>(w, c);
}

// M == 1: one thread per output column; the activation row is staged in LDS.
// The 2^BITS codebook values, computed once per workgroup into LDS (the
// same fp32 values canon() gives per element).
template <int BITS>
__device__ __forceinline__ void canon_table(float* tab) {
  for (int c = threadIdx.x; c < (1 << BITS); c += blockDim.x) tab[c] = canon<BITS>(c);
}

template <int BITS>
__global__ __launch_bounds__(256) void qgemm_f16_m1(F16Args p) {
  extern __shared__ uint16_t arow[];
  __shared__ float tab[1 << BITS];
  for (int k = threadIdx.x; k < p.K; k += 256) arow[k] = p.a[k];
  canon_table<BITS>(tab);
  __syncthreads();
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= p.N) return;  // (after the only barrier)
  // k ascending, one 128-wide group (8 operand chunks of 16 codes) at a
  // time; the next group's codes and scale are loaded while this one runs
  float acc = 0.0f;
  const int ng = p.K / 128;
  uint32_t cur[8][BITS / 2], nxt[8][BITS / 2];
  float sc = group_scale(p, n, 0), sn = sc;
#pragma unroll
  for (int q = 0; q < 8; ++q) raw16<BITS>(p, n, q, cur[q]);
  for (int g = 0; g < ng; ++g) {
    const int gn = min(g + 1, ng - 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) raw16<BITS>(p, n, 8 * gn + q, nxt[q]);
    sn = group_scale(p, n, gn);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      int c[16];
      decode16<BITS>(cur[q], c);
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = fmaf(ifrd::h2f(arow[128 * g + 16 * q + j]), sc * tab[c[j]], acc);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int i = 0; i < BITS / 2; ++i) cur[q][i] = nxt[q][i];
    sc = sn;
  }
  p.out[n] = ifrd::f2h(acc);
}

// M > 1: 64 x 64 outputs per workgroup, 4 x 4 per thread; 32-wide K blocks of
// the activation (fp16) and the dequantized weight (rounded to fp16) staged
// in LDS; each output accumulates its K block's products in ascending k.
template <int BITS>
__global__ __launch_bounds__(256) void qgemm_f16_tiled(F16Args p) {
  constexpr int BM = 64, BN = 64, BK = 32;
  __shared__ uint16_t sA[BM][BK + 2];
  __shared__ uint16_t sW[BN][BK + 2];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int k0 = 0; k0 < p.K; k0 += BK) {
    for (int e = threadIdx.x; e < BM * BK; e += 256) {
      const int r = e / BK, c = e % BK, m = m0 + r;
      sA[r][c] = m < p.M ? p.a[(size_t)m * p.K + k0 + c] : (uint16_t)0;
    }
    if (threadIdx.x < BN * BK / 16) {  // one 16-code chunk of one column each
      const int r = threadIdx.x >> 1, h = threadIdx.x & 1, n = n0 + r;
      if (n < p.N) {
        const int q0 = k0 / 16 + h;
        const float sc = group_scale(p, n, q0 >> 3);
        int c[16];
        codes16<BITS>(p, n, q0, c);
#pragma unroll
        for (int j = 0; j < 16; ++j) sW[r][16 * h + j] = ifrd::f2h(sc * canon<BITS>(c[j]));
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) sW[r][16 * h + j] = 0;
      }
    }
    __syncthreads();
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = ifrd::h2f(sA[ty * 4 + i][kk]);
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = ifrd::h2f(sW[tx * 4 + j][kk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < p.M && n < p.N) p.out[(size_t)m * p.N + n] = ifrd::f2h(acc[i][j]);
    }
}

template <int BITS>
hipError_t launch_f16_bits(const F16Args& p, hipStream_t st) {
  if (p.M == 1) {
    const size_t lds = (size_t)p.K * sizeof(uint16_t);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(qgemm_f16_m1<BITS>, dim3((p.N + 255) / 256), dim3(256), lds, st, p);
  } else {
    hipLaunchKernelGGL(qgemm_f16_tiled<BITS>, dim3((p.N + 63) / 64, (p.M + 63) / 64), dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_qgemm_f16(const F16Args& p, hipStream_t st) {
  if (p.M <= 0) return hipSuccess;
  if (!p.a || !p.codes || !p.sz || !p.out || p.N % 16 != 0 || p.K % 128 != 0 || p.ng != p.K / 128 ||
      p.nsteps != p.K / 64)
    return hipErrorInvalidValue;
  switch (p.bits) {
    case 2: return launch_f16_bits<2>(p, st);
    case 4: return launch_f16_bits<4>(p, st);
    case 8: return launch_f16_bits<8>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ifrk
