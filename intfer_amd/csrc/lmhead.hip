// lm_head (tied embedding) as an int8 x int8 MFMA GEMM fused with a
// first-max-wins argmax.
//
// Weights: per-row symmetric int8 with an fp16 row scale, quantized at load
// exactly as the reference's INT8 lm_head upload (examples/intfer_cli/
// main.cpp:1745-1761).  Activations: final-normed rows quantized per 64-wide
// slice with round-to-nearest-even (the reference lm_head act-quant,
// main.cpp:2445-2451, dashq.hpp:61-78).  Per 64-slice s:
//     T = sum a_q * w_q (int32), acc = fma((float)T, as(m,s), acc)
// logit = acc * ws(v).  Argmax: strict '>' scanning the vocabulary in order
// (main.cpp:8289-8312); ties keep the lower index.
#include "ifr_dev.h"
#include "ifr_kernels.h"

namespace ifrk {
namespace {

constexpr int kWN = 2;  // column tiles per wave

struct LmP {
  const int8_t* a;
  const float* as;
  const uint32_t* w;
  const uint16_t* ws;
  float* logits;
  float* pv;
  int32_t* pi;
  int W, V, H, nsteps;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int WM>
__global__ __launch_bounds__(256) void lmhead_kernel(LmP p) {
  extern __shared__ float as_l[];  // [16 WM rows][nsteps] activation scales of the block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.V >> 4;
  const int part = blockIdx.x * 4 + wave;
  const int tile0 = part * kWN;
  const int row0 = blockIdx.y * 16 * WM;
  int tl[kWN];
#pragma unroll
  for (int j = 0; j < kWN; ++j) tl[j] = min(tile0 + j, ntiles - 1);
  const int8_t* arow[WM];  // A tiles: one 1 KB tile per (16 rows, K step)
#pragma unroll
  for (int i = 0; i < WM; ++i)
    arow[i] = p.a + ((size_t)(min(row0 + 16 * i, p.W - 1) >> 4) * p.nsteps << 10) + 16 * lane;
  // the block's activation scales, staged once (rows past W read row W - 1):
  // per K step a lane then reads its 4 WM scales from LDS instead of memory
  for (int e = threadIdx.x; e < 16 * WM * p.nsteps; e += 256) {
    const int r = e / p.nsteps, s = e - r * p.nsteps;
    as_l[e] = p.as[(size_t)min(row0 + r, p.W - 1) * p.nsteps + s];
  }
  __syncthreads();
  v4f acc[WM][kWN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < kWN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.nsteps; ++s) {
    v4i A[WM], B[kWN];
#pragma unroll
    for (int i = 0; i < WM; ++i) A[i] = *reinterpret_cast<const v4i*>(arow[i] + 1024 * s);
#pragma unroll
    for (int j = 0; j < kWN; ++j)
      B[j] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p.w) +
                                        ((size_t)tl[j] * p.nsteps + s) * 64 + lane);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      float asr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) asr[r] = as_l[(16 * i + 4 * lgrp + r) * p.nsteps + s];
#pragma unroll
      for (int j = 0; j < kWN; ++j) {
        const v4i T = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], B[j], (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf((float)T[r], asr[r], acc[i][j][r]);
      }
    }
  }
  float wsv[kWN];
#pragma unroll
  for (int j = 0; j < kWN; ++j) wsv[j] = ifrd::h2f(p.ws[16 * tl[j] + lrow]);
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 16 * i + 4 * lgrp + r;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < kWN; ++j) {
        const int col = 16 * (tile0 + j) + lrow;
        if (tile0 + j >= ntiles) continue;
        const float lg = acc[i][j][r] * wsv[j];
        if (p.logits && row < p.W) p.logits[(size_t)row * p.V + col] = lg;
        if (better(lg, col, bv, bi)) { bv = lg; bi = col; }
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      if (lrow == 0 && row < p.W) {
        // row-major [row][part] (part count = 4 gridDim.x): the final
        // reduce reads each row's partials contiguously
        const size_t at = (size_t)row * (4 * gridDim.x) + part;
        p.pv[at] = bv;
        p.pi[at] = bi;
      }
    }
}

// Reduce the per-wave (value, index) partials of each row in part order.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float* pv, const int32_t* pi,
                                                           int nparts, int W, int32_t* best) {
  const int row = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int q = threadIdx.x; q < nparts; q += blockDim.x) {
    const float v = pv[(size_t)row * nparts + q];
    const int i = pi[(size_t)row * nparts + q];
    if (better(v, i, bv, bi)) { bv = v; bi = i; }
  }
  __shared__ float sv[256];
  __shared__ int si[256];
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      if (better(sv[threadIdx.x + s], si[threadIdx.x + s], sv[threadIdx.x], si[threadIdx.x])) {
        sv[threadIdx.x] = sv[threadIdx.x + s];
        si[threadIdx.x] = si[threadIdx.x + s];
      }
    }
    __syncthreads();
  }
  // The reference starts from -1e30 with strict '>': a row whose logits are
  // all <= -1e30 reports -1.
  if (threadIdx.x == 0) best[row] = (sv[0] > -1e30f) ? si[0] : -1;
}

template <int WM>
hipError_t launch_wm(const LmP& p, int nparts, int nrb, hipStream_t st) {
  const size_t lds = (size_t)16 * WM * p.nsteps * sizeof(float);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(lmhead_kernel<WM>, dim3(nparts / 4, nrb), dim3(256), lds, st, p);
  return hipGetLastError();
}

}  // namespace

int lmhead_nparts(int V) {
  const int ntiles = V / 16;
  const int waves = (ntiles + kWN - 1) / kWN;
  return ((waves + 3) / 4) * 4;
}

hipError_t launch_lmhead(LmHeadArgs& a, hipStream_t st) {
  if (a.W <= 0) return hipSuccess;
  if (a.V % 16 != 0 || a.H % 64 != 0 || !a.a || !a.as || !a.wcodes || !a.wscale || !a.part_val ||
      !a.part_idx || !a.best)
    return hipErrorInvalidValue;
  a.nparts = lmhead_nparts(a.V);
  LmP p{a.a, a.as, a.wcodes, a.wscale, a.logits, a.part_val, a.part_idx, a.W, a.V, a.H, a.H / 64};
  hipError_t e;
  if (a.W <= 16) e = launch_wm<1>(p, a.nparts, 1, st);
  else if (a.W <= 32) e = launch_wm<2>(p, a.nparts, 1, st);
  else if (a.W <= 64) e = launch_wm<4>(p, a.nparts, 1, st);
  else e = launch_wm<4>(p, a.nparts, (a.W + 63) / 64, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(a.W), dim3(256), 0, st, a.part_val, a.part_idx,
                     a.nparts, a.W, a.best);
  return hipGetLastError();
}

}  // namespace ifrk
