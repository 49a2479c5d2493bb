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

// Code (n, k) of a linear in the fragment-major layout (pack_linear_host):
// column tile n / 16, K step k / 64, lane 16 (k % 64 / 16) + n % 16, code
// j = k % 16 of that lane, operand dword j / 4, byte j % 4.
template <int BITS>
__device__ __forceinline__ int code_at(const uint32_t* codes, int nsteps, int n, int k) {
  const int t = n >> 4, c = n & 15, s = k >> 6, kk = k & 63;
  const int l = 16 * (kk >> 4) + c, j = kk & 15, d = j >> 2, b = j & 3;
  const size_t lane = ((size_t)t * nsteps + s) * 64 + l;
  if constexpr (BITS == 2) return (int)((codes[lane] >> (8 * b + 2 * d)) & 3u);
  else if constexpr (BITS == 4) return (int)((codes[lane * 2 + (d >> 1)] >> (8 * b + 4 * (d & 1))) & 15u);
  else return (int)(((codes[lane * 4 + d] >> (8 * b)) & 0xFFu) ^ 0x80u);  // stored c ^ 0x80
}

template <int BITS>
__device__ __forceinline__ float canon(int c) {
  if constexpr (BITS == 2) {
    return c == 0 ? -1.0f : c == 1 ? -1.0f / 3.0f : c == 2 ? 1.0f / 3.0f : 1.0f;
  } else {
    constexpr float C = (float)((1 << BITS) - 1);
    return (2.0f * (float)c - C) / C;
  }
}

template <int BITS>
__device__ __forceinline__ float weight(const F16Args& p, int n, int k) {
  const uint32_t zw = p.sz[((size_t)(n >> 4) * p.ng + (k >> 7)) * 16 + (n & 15)];
  const float s = ifrd::h2f((uint16_t)(zw & 0xFFFFu)) * p.alpha;
  return s * canon<BITS>(code_at<BITS>(p.codes, p.nsteps, n, k));
}

// M == 1: one thread per output column; the activation row is staged in LDS.
template <int BITS>
__global__ __launch_bounds__(256) void qgemm_f16_m1(F16Args p) {
  extern __shared__ uint16_t arow[];
  for (int k = threadIdx.x; k < p.K; k += 256) arow[k] = p.a[k];
  __syncthreads();
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= p.N) return;  // (after the only barrier)
  float acc = 0.0f;
  for (int k = 0; k < p.K; ++k) acc = fmaf(ifrd::h2f(arow[k]), weight<BITS>(p, n, k), acc);
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
      const int r = e / BK, c = e % BK, m = m0 + r, n = n0 + r;
      sA[r][c] = m < p.M ? p.a[(size_t)m * p.K + k0 + c] : (uint16_t)0;
      sW[r][c] = n < p.N ? ifrd::f2h(weight<BITS>(p, n, k0 + c)) : (uint16_t)0;
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
