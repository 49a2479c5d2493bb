// W2A8 / W4A8 / W8A8 quantized GEMM on gfx950 int8 MFMA with int32 accumulation.
//
// Integer contract (the W2A8 DPAS contract of the reference, dpas48_tiled,
// src/gemm/quant_gemm.cpp:3602-3736, generalized to per-(row,group) scale and
// zero):  for each 128-wide K group g
//     T(m,n,g) = sum_k a_q(m,k) * code(n,k)      exact int32, v_mfma_i32_16x16x64_i8
//     S(m,g)   = sum_k a_q(m,k)                  from the activation producer
//     d   = fma(-zero(n,g), S, T)
//     acc = fma(scale(n,g), d, acc)              groups strictly ascending
// y(m,n) = fp16_rne(ascale(m) * acc).  The fold order is fixed per output
// element: split-K variants exchange the int32 T through LDS and fold them in
// group order, so every launch shape produces the same bits.
//
// Tiling: a workgroup is 4 waves (256 lanes).  Each wave owns WM x WN tiles of
// 16x16 outputs (MFMA 16x16x64).  KSPLIT=1: the 4 waves sit side by side on N
// and each folds its own accumulators (large M, MFMA-bound).  KSPLIT=4: the 4
// waves split the K groups of the same tile and fold after one LDS exchange
// (small M, weight-stream bound).  Codes are read in the fragment-major layout
// below, one fully coalesced 256*bits/8-byte block per (tile, K step).
#include "ifr_dev.h"
#include "ifr_kernels.h"

#include <algorithm>
#include <thread>
#include <vector>

namespace ifrk {
namespace {

constexpr int kG = 128;

// Unpack one lane's codes for one 64-wide K step into the int8 B operand:
// operand dword d holds codes j = 4d..4d+3 in bytes 0..3.
template <int BITS>
__device__ __forceinline__ v4i load_b(const uint32_t* __restrict__ codes, size_t idx) {
  v4i r;
  if constexpr (BITS == 2) {
    const uint32_t w = __builtin_nontemporal_load(codes + idx);
    r.x = (int)(w & 0x03030303u);
    r.y = (int)((w >> 2) & 0x03030303u);
    r.z = (int)((w >> 4) & 0x03030303u);
    r.w = (int)((w >> 6) & 0x03030303u);
  } else if constexpr (BITS == 4) {
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    const v2u w = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(codes) + idx);
    r.x = (int)(w.x & 0x0F0F0F0Fu);
    r.y = (int)((w.x >> 4) & 0x0F0F0F0Fu);
    r.z = (int)(w.y & 0x0F0F0F0Fu);
    r.w = (int)((w.y >> 4) & 0x0F0F0F0Fu);
  } else {
    r = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(codes) + idx);
  }
  return r;
}

// INT8 codes (0..255) are stored as c - 128 so the signed-int8 MFMA sees
// them exactly; the true T is T' + 128 * S (exact in int32).
template <int BITS>
__device__ __forceinline__ int32_t true_t(int32_t t, float S) {
  if constexpr (BITS == 8) return t + 128 * (int32_t)S;
  return t;
}

struct KParams {
  const int8_t* a;
  const float* as;
  const float* gs;
  const uint32_t* codes;
  const uint32_t* sz;
  uint16_t* out;
  int32_t* tdump;
  int M, N, K, ng, nsteps, ldo;
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// Store one finished output element (EPI 0) or a gate/up pair (EPI 1).
__device__ __forceinline__ void store_plain(const KParams& p, int row, int col, float acc) {
  p.out[(size_t)row * p.ldo + col] = ifrd::f2h(p.as[row] * acc);
}
__device__ __forceinline__ void store_swiglu(const KParams& p, int row, int col, float accg,
                                             float accu) {
  const float a = p.as[row];
  const float g = ifrd::fp16r(a * accg);
  const float u = ifrd::fp16r(a * accu);
  p.out[(size_t)row * p.ldo + col] = ifrd::f2h(silu_f(g) * u);
}

template <int BITS, int WM, int WN, int KSPLIT, int EPI>
__global__ __launch_bounds__(256) void qgemm_kernel(KParams p) {
  extern __shared__ int32_t lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.N >> 4;
  const int row0 = blockIdx.y * 16 * WM;
  int tile0, g0, g1;
  if constexpr (KSPLIT == 1) {
    tile0 = (blockIdx.x * 4 + wave) * WN;
    g0 = 0;
    g1 = p.ng;
    if (tile0 >= ntiles) return;  // no barrier in this variant
  } else {
    tile0 = blockIdx.x * WN;
    g0 = (p.ng * wave) / 4;
    g1 = (p.ng * (wave + 1)) / 4;
  }

  const int8_t* arow[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    int r = row0 + 16 * i + lrow;
    r = r < p.M ? r : p.M - 1;
    arow[i] = p.a + (size_t)r * p.K + 16 * lgrp;
  }
  int tl[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) tl[j] = min(tile0 + j, ntiles - 1);

  v4i T[WM][WN];
  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      T[i][j] = (v4i){0, 0, 0, 0};
      acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
    }

  for (int g = g0; g < g1; ++g) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = 2 * g + h;
      v4i A[WM], B[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) A[i] = *reinterpret_cast<const v4i*>(arow[i] + 64 * s);
#pragma unroll
      for (int j = 0; j < WN; ++j)
        B[j] = load_b<BITS>(p.codes, ((size_t)tl[j] * p.nsteps + s) * 64 + lane);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          T[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], B[j], T[i][j], 0, 0, 0);
    }
    if constexpr (KSPLIT == 1) {
      // Fold group g.  C layout: lane holds column lrow, rows 4*lgrp + r.
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const uint32_t szw = p.sz[((size_t)tl[j] * p.ng + g) * 16 + lrow];
        const float sc = ifrd::h2f((uint16_t)(szw & 0xFFFFu));
        const float ze = ifrd::h2f((uint16_t)(szw >> 16));
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int row = row0 + 16 * i + 4 * lgrp + r;
            row = row < p.M ? row : p.M - 1;
            const float S = p.gs[(size_t)row * p.ng + g];
            const int32_t Tv = true_t<BITS>(T[i][j][r], S);
            const float d = fmaf(-ze, S, (float)Tv);
            acc[i][j][r] = fmaf(sc, d, acc[i][j][r]);
            if (p.tdump && row0 + 16 * i + 4 * lgrp + r < p.M && tile0 + j < ntiles)
              p.tdump[((size_t)row * p.N + 16 * tl[j] + lrow) * p.ng + g] = Tv;
          }
          T[i][j] = (v4i){0, 0, 0, 0};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          *reinterpret_cast<v4i*>(&lds[(((size_t)g * WM + i) * WN + j) * 256 + lane * 4]) = T[i][j];
          T[i][j] = (v4i){0, 0, 0, 0};
        }
    }
  }

  if constexpr (KSPLIT == 1) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + 16 * i + 4 * lgrp + r;
        if (row >= p.M) continue;
        if constexpr (EPI == 0) {
#pragma unroll
          for (int j = 0; j < WN; ++j)
            if (tile0 + j < ntiles) store_plain(p, row, 16 * (tile0 + j) + lrow, acc[i][j][r]);
        } else {
#pragma unroll
          for (int j = 0; j < WN; j += 2)
            if (tile0 + j + 1 < ntiles)
              store_swiglu(p, row, 16 * ((tile0 + j) >> 1) + lrow, acc[i][j][r], acc[i][j + 1][r]);
        }
      }
  } else {
    __syncthreads();
    // Fold all groups in order from LDS.  Output o = ((i*WN + j)*64 + lane')*4 + r.
    constexpr int JS = (EPI == 0) ? 1 : 2;  // swiglu: one thread folds the pair
    constexpr int NOUT = WM * (WN / JS) * 256;
    for (int o = threadIdx.x; o < NOUT; o += 256) {
      const int r = o & 3, ln = (o >> 2) & 63, ij = o >> 8;
      const int jj = (ij % (WN / JS)) * JS, i = ij / (WN / JS);
      const int row = row0 + 16 * i + 4 * (ln >> 4) + r;
      const int c = ln & 15;
      float a0 = 0.f, a1 = 0.f;
      const int rr = row < p.M ? row : p.M - 1;
      for (int g = 0; g < p.ng; ++g) {
        const float S = p.gs[(size_t)rr * p.ng + g];
#pragma unroll
        for (int q = 0; q < JS; ++q) {
          const int j = jj + q;
          const int32_t Tv = true_t<BITS>(lds[(((size_t)g * WM + i) * WN + j) * 256 + ln * 4 + r], S);
          const uint32_t szw = p.sz[((size_t)tl[j] * p.ng + g) * 16 + c];
          const float sc = ifrd::h2f((uint16_t)(szw & 0xFFFFu));
          const float ze = ifrd::h2f((uint16_t)(szw >> 16));
          const float d = fmaf(-ze, S, (float)Tv);
          if (q == 0) a0 = fmaf(sc, d, a0); else a1 = fmaf(sc, d, a1);
          if (EPI == 0 && p.tdump && row < p.M && tile0 + j < ntiles)
            p.tdump[((size_t)row * p.N + 16 * tl[j] + c) * p.ng + g] = Tv;
        }
      }
      if (row >= p.M) continue;
      if constexpr (EPI == 0) {
        if (tile0 + jj < ntiles) store_plain(p, row, 16 * (tile0 + jj) + c, a0);
      } else {
        if (tile0 + jj + 1 < ntiles) store_swiglu(p, row, 16 * ((tile0 + jj) >> 1) + c, a0, a1);
      }
    }
  }
}

template <int BITS, int WM, int WN, int KSPLIT, int EPI>
hipError_t launch_cfg(const KParams& p, hipStream_t st) {
  const int ntiles = p.N / 16;
  dim3 grid, block(256);
  size_t lds = 0;
  if (KSPLIT == 1) {
    grid = dim3((ntiles + 4 * WN - 1) / (4 * WN), (p.M + 16 * WM - 1) / (16 * WM));
  } else {
    grid = dim3((ntiles + WN - 1) / WN, (p.M + 16 * WM - 1) / (16 * WM));
    lds = (size_t)p.ng * WM * WN * 256 * sizeof(int32_t);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute(
          reinterpret_cast<const void*>(qgemm_kernel<BITS, WM, WN, KSPLIT, EPI>),
          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
  }
  hipLaunchKernelGGL((qgemm_kernel<BITS, WM, WN, KSPLIT, EPI>), grid, block, lds, st, p);
  return hipGetLastError();
}

template <int BITS, int EPI>
hipError_t launch_bits(const KParams& p, hipStream_t st) {
  constexpr int WNs = EPI == 0 ? 1 : 2;
  if (p.M <= 16) return launch_cfg<BITS, 1, WNs, 4, EPI>(p, st);
  if (p.M <= 32) return launch_cfg<BITS, 2, WNs, 4, EPI>(p, st);
  if (p.M <= 64 && p.ng <= (EPI == 0 ? 24 : 16)) return launch_cfg<BITS, 4, WNs, 4, EPI>(p, st);
  return launch_cfg<BITS, 2, 2, 1, EPI>(p, st);
}

}  // namespace

void pack_linear_host(const uint8_t* codes, const uint16_t* scale, const uint16_t* zero, int N,
                      int K, int bits, uint32_t* out_codes, uint32_t* out_sz, int tile_stride,
                      int tile_offset, uint32_t xor8) {
  const int ntiles = N / 16, nsteps = K / 64, ng = K / kG, W = bits / 2;
  auto code_at = [&](size_t n, size_t k) -> uint32_t {
    const size_t i = n * (size_t)K + k;
    if (bits == 8) return codes[i];
    if (bits == 4) return (codes[i / 2] >> ((i % 2) * 4)) & 0xFu;
    return (codes[i / 4] >> ((i % 4) * 2)) & 0x3u;
  };
  auto work = [&](int t0, int t1) {
    for (int t = t0; t < t1; ++t) {
      const size_t td = (size_t)t * tile_stride + tile_offset;
      for (int s = 0; s < nsteps; ++s)
        for (int l = 0; l < 64; ++l) {
          const size_t n = 16 * (size_t)t + (l & 15);
          const size_t kb = 64 * (size_t)s + 16 * (l >> 4);
          uint32_t w[4] = {0, 0, 0, 0};
          for (int j = 0; j < 16; ++j) {
            const uint32_t c = code_at(n, kb + j);
            const int d = j >> 2, b = j & 3;
            if (bits == 2) w[0] |= c << (8 * b + 2 * d);
            else if (bits == 4) w[d >> 1] |= c << (8 * b + 4 * (d & 1));
            else w[d] |= (c ^ xor8) << (8 * b);
          }
          uint32_t* dst = out_codes + ((td * nsteps + s) * 64 + l) * W;
          for (int q = 0; q < W; ++q) dst[q] = w[q];
        }
      if (out_sz)
      for (int g = 0; g < ng; ++g)
        for (int c = 0; c < 16; ++c) {
          const size_t n = 16 * (size_t)t + c;
          out_sz[(td * ng + g) * 16 + c] =
              (uint32_t)scale[n * ng + g] | ((uint32_t)zero[n * ng + g] << 16);
        }
    }
  };
  const int nth = std::max(1, std::min<int>(16, (int)std::thread::hardware_concurrency()));
  if (ntiles < 64 || nth == 1) { work(0, ntiles); return; }
  std::vector<std::thread> th;
  for (int i = 0; i < nth; ++i) {
    const int a = (int)((long)ntiles * i / nth), b = (int)((long)ntiles * (i + 1) / nth);
    th.emplace_back(work, a, b);
  }
  for (auto& t : th) t.join();
}

hipError_t launch_qgemm(const DLin& w, const QGemmArgs& a, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (w.K % kG != 0 || w.N % 16 != 0 || !w.codes || !a.a || !a.as || !a.gs || !a.out)
    return hipErrorInvalidValue;
  if (w.pair && (w.N % 32 != 0 || a.tdump)) return hipErrorInvalidValue;
  KParams p{a.a, a.as, a.gs, w.codes, w.sz, a.out, a.tdump, a.M, w.N, w.K, w.ng, w.nsteps, a.ldo};
  const int epi = w.pair ? 1 : 0;
  switch (w.bits * 2 + epi) {
    case 4: return launch_bits<2, 0>(p, st);
    case 5: return launch_bits<2, 1>(p, st);
    case 8: return launch_bits<4, 0>(p, st);
    case 9: return launch_bits<4, 1>(p, st);
    case 16: return launch_bits<8, 0>(p, st);
    case 17: return launch_bits<8, 1>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ifrk
