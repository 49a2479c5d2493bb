// Row-wise kernels of the mixed-batch forward on gfx950:
//   row_quant   : [embed gather | residual += FWHT(y)/sqrt(K)] -> RMSNorm(1+w)
//                 -> FWHT/sqrt(K) -> per-token (or GA64) int8 quantization
//                 + per-128-group code sums (the S of the GEMM contract)
//   quant_plain : per-token int8 quantization of an fp32/fp16 row
//   qk_rope_kv  : per-head q/k RMSNorm(1+w) + rotate-half RoPE + fp16 round,
//                 Q store, K/V append to the paged cache (fp16 or int8)
//   pack        : ragged batch -> cu_seqlens, row maps, attention work units
// One workgroup per row; the arithmetic follows the reference host helpers
// operation for operation so the results are bit-identical to the CPU oracle
// (RMSNorm in the reference's 8-lane fused order, main.cpp:306-351; FWHT in
// the reference stage order, src/spinquant.cpp:303-312; act-quant with
// correctly rounded division, dashq.cpp:221-336).
#include "ifr_dev.h"
#include "ifr_kernels.h"

#include <algorithm>

namespace ifrk {
namespace {

__device__ __forceinline__ float block_max(float v, float* red) {
  v = ifrd::wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, red[i]);
  return r;
}

// RMSNorm factor over x[0..n) (n a multiple of 8) in the reference AVX2 order:
// eight fused lane accumulators, lanes folded (j, j+4), then two horizontal
// adds.  Called by all threads; returns v = 1/sqrt(sum/n + eps) to all.
__device__ float rms_factor(const float* x, int n, float eps, float* red) {
  __syncthreads();
  if (threadIdx.x < 8) {
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n; i += 8) acc = fmaf(x[i], x[i], acc);
    red[threadIdx.x] = acc;
  }
  __syncthreads();
  const float s0 = red[0] + red[4], s1 = red[1] + red[5], s2 = red[2] + red[6], s3 = red[3] + red[7];
  const float tot = (s0 + s1) + (s2 + s3);
  const float v = 1.0f / sqrtf(tot / (float)n + eps);
  __syncthreads();
  return v;
}

// In-place FWHT of x[0..p) (p a power of two) in the reference stage order,
// then x *= 1/sqrt(p).
__device__ void fwht_lds(float* x, int p) {
  for (int len = 2; len <= p; len <<= 1) {
    const int half = len >> 1;
    __syncthreads();
    for (int b = threadIdx.x; b < (p >> 1); b += blockDim.x) {
      const int i = (b / half) * len + (b % half);
      const float u = x[i], v = x[i + half];
      x[i] = u + v;
      x[i + half] = u - v;
    }
  }
  __syncthreads();
  const float inv = 1.0f / sqrtf((float)p);
  for (int i = threadIdx.x; i < p; i += blockDim.x) x[i] *= inv;
  __syncthreads();
}

__device__ __forceinline__ int floor_pow2(int n) {
  int p = 1;
  while (p * 2 <= n) p *= 2;
  return p;
}

// Quantize x[0..K) held in LDS.  Per row (ga == 0) or per ga-slice.
__device__ void quant_lds(const float* x, int K, int ga, int round, int8_t* q, int m, float* qs,
                          float* gsum, float* red, int* codes_lds) {
  if (ga == 0) {
    float mx = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) mx = fmaxf(mx, fabsf(x[i]));
    mx = fmaxf(1e-6f, block_max(mx, red));
    const float s = mx / 127.0f;
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) qs[0] = s;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      const int c = round == 0 ? ifrd::quant_half_away(x[i], inv) : ifrd::quant_rne(x[i], inv);
      q[atile_off(m, i, K)] = (int8_t)c;
      codes_lds[i] = c;
    }
  } else {
    const int ns = K / ga;
    __syncthreads();
    for (int sl = threadIdx.x; sl < ns; sl += blockDim.x) {
      float mx = 1e-6f;
      for (int k = sl * ga; k < (sl + 1) * ga; ++k) mx = fmaxf(mx, fabsf(x[k]));
      const float s = mx / 127.0f;
      red[64 + sl] = 1.0f / s;
      qs[sl] = s;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      const float inv = red[64 + i / ga];
      const int c = round == 0 ? ifrd::quant_half_away(x[i], inv) : ifrd::quant_rne(x[i], inv);
      q[atile_off(m, i, K)] = (int8_t)c;
      codes_lds[i] = c;
    }
  }
  if (gsum) {
    __syncthreads();
    for (int g = threadIdx.x; g < K / 128; g += blockDim.x) {
      int S = 0;
      for (int k = g * 128; k < g * 128 + 128; ++k) S += codes_lds[k];
      gsum[g] = (float)S;
    }
  }
}

__global__ __launch_bounds__(256) void row_quant_kernel(RowQuantArgs a) {
  extern __shared__ float sh[];
  float* x = sh;                                  // K floats
  int* codes = reinterpret_cast<int*>(sh + a.K);  // K ints
  float* red = sh + 2 * a.K;                      // 64 + K/64 floats
  const int m = blockIdx.x, K = a.K;
  const int src = a.rowmap ? a.rowmap[m] : m;
  if (a.src == SRC_X) {
    for (int i = threadIdx.x; i < K; i += blockDim.x) x[i] = a.x[(size_t)src * K + i];
  } else if (a.src == SRC_EMBED) {
    const float* e = a.embed + (size_t)a.tokens[src] * K;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      const float v = e[i];
      x[i] = v;
      a.resid[(size_t)src * K + i] = v;
    }
  } else {
    for (int i = threadIdx.x; i < K; i += blockDim.x) x[i] = ifrd::h2f(a.y[(size_t)src * K + i]);
    if (a.rot_y) fwht_lds(x, floor_pow2(K));
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
      const float v = a.resid[(size_t)src * K + i] + x[i];
      a.resid[(size_t)src * K + i] = v;
      x[i] = v;
    }
  }
  __syncthreads();
  if (a.norm_w) {
    const float v = rms_factor(x, K, a.eps, red);
    for (int i = threadIdx.x; i < K; i += blockDim.x) x[i] = (x[i] * v) * (1.0f + a.norm_w[i]);
  }
  if (a.rotate) fwht_lds(x, floor_pow2(K));
  __syncthreads();
  const int ns = a.ga ? K / a.ga : 1;
  quant_lds(x, K, a.ga, a.round, a.q, m, a.qscale + (size_t)m * ns,
            a.gsum ? a.gsum + (size_t)m * (K / 128) : nullptr, red, codes);
}

// ---- fast path: K = 1024 rows, 8 waves per row, 2 contiguous elements per thread
//
// FWHT stages in the reference order (half = 1, 2, ..., 512): half 1 inside a
// thread, half 2-64 across lanes of a wave (partner lane ^ half/2), half
// 128-512 through one LDS exchange across the eight waves.  Every output is
// formed by the same adds on the same operands as the sequential loop, so the
// result is bit-identical.
template <int M>
__device__ __forceinline__ float bfly_lane(float x) {
  const float o = ifrd::lane_xor<M>(x);
  return (threadIdx.x & M) ? (o - x) : (x + o);
}

__device__ void fwht1024(float (&v)[2], float* xs) {
  {
    const float a = v[0], b = v[1];
    v[0] = a + b;
    v[1] = a - b;
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<1>(v[e]);
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<2>(v[e]);
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<4>(v[e]);
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<8>(v[e]);
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<16>(v[e]);
#pragma unroll
  for (int e = 0; e < 2; ++e) v[e] = bfly_lane<32>(v[e]);
  __syncthreads();
  *reinterpret_cast<float2*>(xs + 2 * threadIdx.x) = make_float2(v[0], v[1]);
  __syncthreads();
  // element 2 t + e sits in 128-block kb = wave; the last three stages combine
  // the eight blocks' values at the same offset: (a_k = x_k +- x_k^1), then
  // (b = a_k +- a_k^2), then (c = b_k +- b_k^4), each with the reference's
  // operand order, for the one output kb
  const int kb = threadIdx.x >> 6;
  const float inv = 1.0f / sqrtf(1024.0f);
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int off = (2 * threadIdx.x + e) & 127;
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = xs[off + 128 * k];
    // the four stage-128 pairs feeding output kb: pairs (b4 + 2 j2 + {0,1}) for
    // j2 in {0,1} and b4 in {0,4}; keep a_k with k = 2 q + (kb & 1)
    float a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = x[2 * q], hi = x[2 * q + 1];
      a[q] = (kb & 1) ? lo - hi : lo + hi;
    }
    // stage 256: b over (a_q, a_q+1) within each half: b_k with (k & 2) = kb & 2
    const float b0 = (kb & 2) ? a[0] - a[1] : a[0] + a[1];
    const float b1 = (kb & 2) ? a[2] - a[3] : a[2] + a[3];
    // stage 512
    const float c = (kb & 4) ? b0 - b1 : b0 + b1;
    v[e] = c * inv;
  }
}

// RMSNorm factor of the 1024 values held 2 per thread, reference order: eight
// sequential fused chains over x[j + 8n], folded (j, j+4) then two horizontal
// adds.  The row is stored chain-major (chain j = i % 8 holds x[j + 8n] at
// 132 j + n; the stride 132 keeps the stores on distinct banks), so each
// chain reads its 128 values 4 at a time.
constexpr int kRms1024Lds = 8 * 132;  // floats of xs the chain-major copy uses
__device__ float rms1024(const float (&v)[2], float* xs, float* red, float eps) {
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int i = 2 * threadIdx.x + e;
    xs[(i & 7) * 132 + (i >> 3)] = v[e];
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    float acc = 0.0f;
    const float4* xc = reinterpret_cast<const float4*>(xs + threadIdx.x * 132);
#pragma unroll
    for (int n4 = 0; n4 < 32; n4 += 8) {
      float4 x8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x8[i] = xc[n4 + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc = fmaf(x8[i].x, x8[i].x, acc);
        acc = fmaf(x8[i].y, x8[i].y, acc);
        acc = fmaf(x8[i].z, x8[i].z, acc);
        acc = fmaf(x8[i].w, x8[i].w, acc);
      }
    }
    red[threadIdx.x] = acc;
  }
  __syncthreads();
  const float s0 = red[0] + red[4], s1 = red[1] + red[5], s2 = red[2] + red[6], s3 = red[3] + red[7];
  const float tot = (s0 + s1) + (s2 + s3);
  return 1.0f / sqrtf(tot / 1024.0f + eps);
}

__global__ __launch_bounds__(512) void row_quant1024_kernel(RowQuantArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kRms1024Lds];  // fwht1024 uses the first 1024
  __shared__ float red[16];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int src = a.rowmap ? a.rowmap[m] : m;
  float v[2];
  if (a.src == SRC_X) {
    const float2 x2 = *reinterpret_cast<const float2*>(a.x + (size_t)src * 1024 + 2 * t);
    v[0] = x2.x; v[1] = x2.y;
  } else if (a.src == SRC_EMBED) {
    const float2 x2 = *reinterpret_cast<const float2*>(a.embed + (size_t)a.tokens[src] * 1024 + 2 * t);
    v[0] = x2.x; v[1] = x2.y;
    *reinterpret_cast<float2*>(a.resid + (size_t)src * 1024 + 2 * t) = x2;
  } else {
    // both loads issued together: the residual does not wait behind the
    // rotation's barriers
    const uint32_t y2 = *reinterpret_cast<const uint32_t*>(a.y + (size_t)src * 1024 + 2 * t);
    float2* rp = reinterpret_cast<float2*>(a.resid + (size_t)src * 1024 + 2 * t);
    float2 r2 = *rp;
    v[0] = ifrd::h2f((uint16_t)(y2 & 0xFFFF));
    v[1] = ifrd::h2f((uint16_t)(y2 >> 16));
    if (a.rot_y) fwht1024(v, xs);
    r2.x = r2.x + v[0]; r2.y = r2.y + v[1];
    *rp = r2;
    v[0] = r2.x; v[1] = r2.y;
  }
  if (a.norm_w) {
    const float f = rms1024(v, xs, red, a.eps);
    const float2 w2 = *reinterpret_cast<const float2*>(a.norm_w + 2 * t);
    v[0] = (v[0] * f) * (1.0f + w2.x);
    v[1] = (v[1] * f) * (1.0f + w2.y);
  }
  if (a.rotate) fwht1024(v, xs);
  int c[2];
  if (a.ga == 0) {
    float mx = fmaxf(fabsf(v[0]), fabsf(v[1]));
    mx = ifrd::wave_max(mx);
    __syncthreads();
    if (lane == 0) red[8 + (t >> 6)] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(fmaxf(red[8], red[9]), fmaxf(red[10], red[11])),
               fmaxf(fmaxf(red[12], red[13]), fmaxf(red[14], red[15])));
    mx = fmaxf(1e-6f, mx);
    const float s = mx / 127.0f;
    const float inv = 1.0f / s;
    if (t == 0) a.qscale[m] = s;
#pragma unroll
    for (int e = 0; e < 2; ++e)
      c[e] = a.round == 0 ? ifrd::quant_half_away(v[e], inv) : ifrd::quant_rne(v[e], inv);
  } else {  // 64-wide slices = 32 lanes
    float mx = fmaxf(fabsf(v[0]), fabsf(v[1]));
    mx = ifrd::row16_max(mx);
    mx = fmaxf(1e-6f, fmaxf(mx, ifrd::lane_xor<16>(mx)));
    const float s = mx / 127.0f;
    const float inv = 1.0f / s;
    if ((lane & 31) == 0) a.qscale[(size_t)m * 16 + (t >> 5)] = s;
#pragma unroll
    for (int e = 0; e < 2; ++e)
      c[e] = a.round == 0 ? ifrd::quant_half_away(v[e], inv) : ifrd::quant_rne(v[e], inv);
  }
  const uint16_t packed = (uint16_t)((uint32_t)(c[0] & 0xFF) | ((uint32_t)(c[1] & 0xFF) << 8));
  *reinterpret_cast<uint16_t*>(a.q + atile_off(m, 2 * t, 1024)) = packed;
  if (a.gsum) {  // 128-wide groups = one wave (integer sums: order-free)
    const int S = ifrd::wave_sum_int(c[0] + c[1]);
    if (lane == 0) a.gsum[(size_t)m * 8 + (t >> 6)] = (float)S;
  }
}

// ---- any K (a multiple of 256, up to 8192): the row in registers -----------
//
// The row splits into the power-of-two head [0, P) the FWHT rotates
// (blockdiag(H_P, I), spinquant.cpp:586-604) and the tail [P, K).  Thread t
// holds the E = P / 256 contiguous head elements [E t, E t + E) and the
// ET = (K - P) / 256 contiguous tail elements [P + ET t, +ET).  FWHT stages
// in the reference order: half < E inside the thread, half = E .. 32 E across
// the lanes of a wave (partner lane ^ half / E), the last two (half = P / 4,
// P / 2, across the four waves) through one LDS exchange, as fwht1024 does.
// Every output is formed by the same adds on the same operands as the
// sequential loop, and the RMS sum runs the reference's eight sequential
// chains over the LDS copy of the row, so the result is bit-identical to the
// LDS kernel it replaces.
template <int M, int E>
__device__ __forceinline__ void bfly_lanes(float (&v)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = bfly_lane<M>(v[e]);
}

// LDS index of row element i with one pad float per 32: lanes that hold E
// consecutive elements each (E a power of two) then hit 32 distinct banks
// instead of a few.
__device__ __forceinline__ int pad32(int i) { return i + (i >> 5); }

template <int E>
__device__ void fwht_regs(float (&v)[E], float* xs) {
  constexpr int P = 256 * E;
#pragma unroll
  for (int half = 1; half < E; half <<= 1)
#pragma unroll
    for (int e = 0; e < E; ++e)
      if ((e & half) == 0) {
        const float a = v[e], b = v[e + half];
        v[e] = a + b;
        v[e + half] = a - b;
      }
  bfly_lanes<1>(v);
  bfly_lanes<2>(v);
  bfly_lanes<4>(v);
  bfly_lanes<8>(v);
  bfly_lanes<16>(v);
  bfly_lanes<32>(v);
  __syncthreads();
#pragma unroll
  for (int e = 0; e < E; ++e) xs[pad32(E * threadIdx.x + e)] = v[e];
  __syncthreads();
  const int q = threadIdx.x >> 6;  // quarter of the P head elements
  const float inv = 1.0f / sqrtf((float)P);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int base = (E * threadIdx.x + e) & (P / 4 - 1);
    const float a0 = xs[pad32(base)], a1 = xs[pad32(base + P / 4)], a2 = xs[pad32(base + P / 2)],
                a3 = xs[pad32(base + 3 * P / 4)];
    const float b0 = a0 + a1, b1 = a0 - a1, b2 = a2 + a3, b3 = a2 - a3;
    const float c = q == 0 ? b0 + b2 : q == 1 ? b1 + b3 : q == 2 ? b0 - b2 : b1 - b3;
    v[e] = c * inv;
  }
}

// n (<= N) contiguous fp32 values between p and r: 16-byte accesses when n
// is a multiple of 4 (p is then 16-byte aligned), single floats otherwise,
// never past p[n - 1].
template <int N>
__device__ __forceinline__ void ld_f32(const float* p, float* r, int n) {
  if (N % 4 == 0 && n % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      if (4 * i >= n) break;
      const float4 x = reinterpret_cast<const float4*>(p)[i];
      r[4 * i] = x.x; r[4 * i + 1] = x.y; r[4 * i + 2] = x.z; r[4 * i + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < n) r[i] = p[i];
  }
}
template <int N>
__device__ __forceinline__ void st_f32(float* p, const float* r, int n) {
  if (N % 4 == 0 && n % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      if (4 * i >= n) break;
      reinterpret_cast<float4*>(p)[i] = make_float4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < n) p[i] = r[i];
  }
}
template <int N>
__device__ __forceinline__ void ld_f16(const uint16_t* p, float* r, int n) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (i < n) r[i] = ifrd::h2f(p[i]);
}

// Sum over aligned groups of n lanes (n a power of two; n > 64: the whole wave).
__device__ __forceinline__ int group_lanes_sum(int v, int n) {
  for (int off = 1; off < n && off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float group_lanes_max(float v, int n) {
  for (int off = 1; off < n && off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// n (<= N) int8 codes for the consecutive columns k0.. of row m, k0 a multiple
// of min(n, 16): whole 16-byte lane chunks where n >= 16, else one 4- or
// 8-byte piece of a chunk, else single bytes.
template <int N>
__device__ __forceinline__ void store_codes(int8_t* q, int m, int k0, int K, const int* c, int n) {
  if (n >= 16) {
#pragma unroll
    for (int j = 0; j < N / 16; ++j) {
      if (16 * j >= n) break;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t)(c[16 * j + i] & 0xFF) << (8 * (i & 3));
      *reinterpret_cast<uint4*>(q + atile_off(m, k0 + 16 * j, K)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else if (n == 8 || n == 4) {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < (N < 8 ? N : 8); ++i)
      if (i < n) w[i >> 2] |= (uint32_t)(c[i] & 0xFF) << (8 * (i & 3));
    if (n == 8) *reinterpret_cast<uint2*>(q + atile_off(m, k0, K)) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(q + atile_off(m, k0, K)) = w[0];
  } else {
#pragma unroll
    for (int i = 0; i < (N < 4 ? N : 4); ++i)
      if (i < n) q[atile_off(m, k0 + i, K)] = (int8_t)c[i];
  }
}

template <int E>
__global__ __launch_bounds__(256) void row_quant_wide(RowQuantArgs a) {
  // the padded FWHT exchange (P + P / 32) or the chain-major row (K + 32)
  __shared__ __attribute__((aligned(16))) float xs[8192 + 256];
  __shared__ float red[16];
  constexpr int P = 256 * E;
  const int K = a.K, ET = (K - P) / 256;
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int src = a.rowmap ? a.rowmap[m] : m;
  const size_t h0 = (size_t)src * K + (size_t)E * t, t0 = (size_t)src * K + P + (size_t)ET * t;
  float v[E], w[E];  // head, tail (ET <= E - 1 values used)
#pragma unroll
  for (int e = 0; e < E; ++e) w[e] = 0.0f;
  if (a.src == SRC_X) {
    ld_f32<E>(a.x + h0, v, E);
    ld_f32<E>(a.x + t0, w, ET);
  } else if (a.src == SRC_EMBED) {
    const float* er = a.embed + (size_t)a.tokens[src] * K;
    ld_f32<E>(er + (size_t)E * t, v, E);
    ld_f32<E>(er + P + (size_t)ET * t, w, ET);
    st_f32<E>(a.resid + h0, v, E);
    st_f32<E>(a.resid + t0, w, ET);
  } else {
    float rv[E], rw[E];
    ld_f32<E>(a.resid + h0, rv, E);
    ld_f32<E>(a.resid + t0, rw, ET);
    ld_f16<E>(a.y + h0, v, E);
    ld_f16<E>(a.y + t0, w, ET);
    if (a.rot_y) fwht_regs<E>(v, xs);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      v[e] = rv[e] + v[e];
      w[e] = rw[e] + w[e];
    }
    st_f32<E>(a.resid + h0, v, E);
    st_f32<E>(a.resid + t0, w, ET);
  }
  if (a.norm_w) {
    // The row in LDS chain-major for the eight sequential chains
    // (rms_factor's order): chain j = i % 8 holds x[j + 8 n] at j * CS + n,
    // so each chain reads its values 4 at a time in order.  K / 8 is a
    // multiple of 32 (K a multiple of 256), CS a multiple of 4.
    const int CS = K / 8 + 4;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = E * t + e;
      xs[(i & 7) * CS + (i >> 3)] = v[e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (e < ET) {
        const int i = P + ET * t + e;
        xs[(i & 7) * CS + (i >> 3)] = w[e];
      }
    __syncthreads();
    if (t < 8) {
      float acc = 0.0f;
      const float4* xc = reinterpret_cast<const float4*>(xs + t * CS);
      for (int n4 = 0; n4 < K / 32; n4 += 8) {
        float4 x8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x8[i] = xc[n4 + i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc = fmaf(x8[i].x, x8[i].x, acc);
          acc = fmaf(x8[i].y, x8[i].y, acc);
          acc = fmaf(x8[i].z, x8[i].z, acc);
          acc = fmaf(x8[i].w, x8[i].w, acc);
        }
      }
      red[t] = acc;
    }
    __syncthreads();
    const float s0 = red[0] + red[4], s1 = red[1] + red[5], s2 = red[2] + red[6], s3 = red[3] + red[7];
    const float tot = (s0 + s1) + (s2 + s3);
    const float f = 1.0f / sqrtf(tot / (float)K + a.eps);
    float nv[E], nw[E];
    ld_f32<E>(a.norm_w + (size_t)E * t, nv, E);
    ld_f32<E>(a.norm_w + P + (size_t)ET * t, nw, ET);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      v[e] = (v[e] * f) * (1.0f + nv[e]);
      if (e < ET) w[e] = (w[e] * f) * (1.0f + nw[e]);
    }
  }
  if (a.rotate) fwht_regs<E>(v, xs);
  // quantization: per row (ga 0) or per 64-wide slice (ga 64)
  float sh_ = 0.0f, st_ = 0.0f;  // scale of the head / tail element slices
  float ih = 0.0f, it = 0.0f;
  if (a.ga == 0) {
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      mx = fmaxf(mx, fabsf(v[e]));
      if (e < ET) mx = fmaxf(mx, fabsf(w[e]));
    }
    mx = ifrd::wave_max(mx);
    __syncthreads();
    if (lane == 0) red[8 + (t >> 6)] = mx;
    __syncthreads();
    mx = fmaxf(1e-6f, fmaxf(fmaxf(red[8], red[9]), fmaxf(red[10], red[11])));
    sh_ = st_ = mx / 127.0f;
    ih = it = 1.0f / sh_;
    if (t == 0) a.qscale[m] = sh_;
  } else {
    // a 64-wide slice is 64 / E head lanes or 64 / ET tail lanes: reduce
    // over aligned groups of that many lanes (E, ET powers of two here)
    float mh = 0.0f, mt = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      mh = fmaxf(mh, fabsf(v[e]));
      if (e < ET) mt = fmaxf(mt, fabsf(w[e]));
    }
    mh = group_lanes_max(mh, 64 / E);
    if (ET > 0) mt = group_lanes_max(mt, 64 / ET);
    mh = fmaxf(1e-6f, mh);
    mt = fmaxf(1e-6f, mt);
    sh_ = mh / 127.0f;
    st_ = mt / 127.0f;
    ih = 1.0f / sh_;
    it = 1.0f / st_;
    if ((E * t) % 64 == 0) a.qscale[(size_t)m * (K / 64) + (E * t) / 64] = sh_;
    if (ET > 0 && (ET * t) % 64 == 0) a.qscale[(size_t)m * (K / 64) + (P + ET * t) / 64] = st_;
  }
  int ch[E], ctl[E];
  int Sh = 0, St = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ch[e] = a.round == 0 ? ifrd::quant_half_away(v[e], ih) : ifrd::quant_rne(v[e], ih);
    Sh += ch[e];
    ctl[e] = 0;
    if (e < ET) {
      ctl[e] = a.round == 0 ? ifrd::quant_half_away(w[e], it) : ifrd::quant_rne(w[e], it);
      St += ctl[e];
    }
  }
  // A-tile stores: the E head codes of a thread are E consecutive columns
  // starting at a multiple of E, inside one 16-byte lane chunk (E <= 16) or
  // spanning E / 16 chunks
  store_codes<E>(a.q, m, E * t, K, ch, E);
  store_codes<E>(a.q, m, P + ET * t, K, ctl, ET);
  if (a.gsum) {  // 128-wide groups: 128 / E head lanes, 128 / ET tail lanes
    Sh = group_lanes_sum(Sh, 128 / E);
    if (ET > 0) St = group_lanes_sum(St, 128 / ET);
    __syncthreads();
    int* sred = reinterpret_cast<int*>(xs);
    if (lane == 0) {  // per-wave sums, for groups of 128 lanes (E or ET = 1)
      sred[t >> 6] = Sh;
      sred[8 + (t >> 6)] = St;
    }
    __syncthreads();
    if ((E * t) % 128 == 0)
      a.gsum[(size_t)m * (K / 128) + (E * t) / 128] =
          (float)(128 / E > 64 ? sred[t >> 6] + sred[(t >> 6) + 1] : Sh);
    if (ET > 0 && (ET * t) % 128 == 0)
      a.gsum[(size_t)m * (K / 128) + (P + ET * t) / 128] =
          (float)(128 / ET > 64 ? sred[8 + (t >> 6)] + sred[8 + (t >> 6) + 1] : St);
  }
}

// Per-token int8 quantization of an fp32 / fp16 row of K = 8 * NT values:
// thread t owns the 8 contiguous columns 8t..8t+7, so its input is one
// 16-byte (fp16) or two 16-byte (fp32) loads, its codes are one 8-byte A-tile
// store, and a 128-column group is exactly one 16-lane DPP row.
template <int NT>
__global__ __launch_bounds__(NT) void quant_plain8(const float* xf, const uint16_t* xh, int8_t* q, float* qs,
                                                   float* gsum) {
  constexpr int K = 8 * NT, NW = NT / 64;
  __shared__ float red[NW];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
  float v[8];
  if (xf) {
    const float4* p = reinterpret_cast<const float4*>(xf + (size_t)m * K + 8 * t);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(xh + (size_t)m * K + 8 * t);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = ifrd::h2f((uint16_t)(w[i] & 0xFFFF));
      v[2 * i + 1] = ifrd::h2f((uint16_t)(w[i] >> 16));
    }
  }
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
  mx = ifrd::wave_max(mx);
  if (lane == 0) red[t >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) mx = fmaxf(mx, red[i]);
  mx = fmaxf(1e-6f, mx);
  const float s = mx / 127.0f;
  const float inv = 1.0f / s;
  if (t == 0) qs[m] = s;
  uint32_t w[2] = {0u, 0u};
  int S = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = ifrd::quant_half_away(v[i], inv);
    w[i >> 2] |= (uint32_t)(c & 0xFF) << (8 * (i & 3));
    S += c;
  }
  *reinterpret_cast<uint2*>(q + atile_off(m, 8 * t, K)) = make_uint2(w[0], w[1]);
  S = ifrd::row16_sum_int(S);
  if (gsum && (lane & 15) == 0) gsum[(size_t)m * (K / 128) + (t >> 4)] = (float)S;
}

// Any K (a multiple of 128, up to 2048 * CH): 256 threads per row, thread t
// holds the 8-element chunks t, t + 256, ... in registers, so the row is read
// once and each chunk is written as one 8-byte A-tile store.  The 16 chunks
// of a 128-column group sit on the 16 lanes of one DPP row, whatever the
// round, because 256 is a multiple of 16.  Same rule as quant_plain8.
template <int CH>
__global__ __launch_bounds__(256) void quant_plain_wide(const float* xf, const uint16_t* xh, int K,
                                                        int8_t* q, float* qs, float* gsum) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int nch = K / 8;
  float v[CH][8];
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = t + 256 * i;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    if (c < nch) {
      if (xf) {
        const float4* p = reinterpret_cast<const float4*>(xf + (size_t)m * K + 8 * c);
        const float4 a = p[0], b = p[1];
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
      } else {
        const uint4 r = *reinterpret_cast<const uint4*>(xh + (size_t)m * K + 8 * c);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[i][2 * e] = ifrd::h2f((uint16_t)(w[e] & 0xFFFF));
          v[i][2 * e + 1] = ifrd::h2f((uint16_t)(w[e] >> 16));
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[i][e]));
  }
  mx = ifrd::wave_max(mx);
  if (lane == 0) red[t >> 6] = mx;
  __syncthreads();
  mx = fmaxf(1e-6f, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  const float s = mx / 127.0f;
  const float inv = 1.0f / s;
  if (t == 0) qs[m] = s;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = t + 256 * i;
    uint32_t w[2] = {0u, 0u};
    int S = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int cq = ifrd::quant_half_away(v[i][e], inv);
      w[e >> 2] |= (uint32_t)(cq & 0xFF) << (8 * (e & 3));
      S += cq;
    }
    S = ifrd::row16_sum_int(S);  // every lane takes part (DPP)
    if (c < nch) {
      *reinterpret_cast<uint2*>(q + atile_off(m, 8 * c, K)) = make_uint2(w[0], w[1]);
      if (gsum && (lane & 15) == 0) gsum[(size_t)m * (K / 128) + (c >> 4)] = (float)S;
    }
  }
}

// ---- q/k norm + RoPE + KV append --------------------------------------------
// grid (M, ceil(heads / 4)): one wave per head vector (hd = 128, 2 dims per lane).
__global__ __launch_bounds__(256) void qk_rope_kv_kernel(QKArgs a, KVLayout kv) {
  __shared__ float hx[4][128];
  __shared__ float red[4][8];
  const int m = blockIdx.x, lane = threadIdx.x & 63;
  // wave-uniform head: the row record, block-table entry and head kind are
  // scalar loads / values
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hd = kv.hd, nq = a.nq, nkv = kv.nkv;
  const int h = blockIdx.y * 4 + w;
  const int nhead = (a.gated ? 2 * nq : nq) + 2 * nkv;  // head-sized column blocks
  if (h >= nhead) return;  // no block-wide barrier below
  const int ncols = nhead * hd;
  const int pos = a.row_pos[m], seq = a.row_seq[m];
  const int half = a.rotary / 2;
  float* x = hx[w];
  int kind, hh;  // q, k, v or gate
  qkv_block(h, nq, nkv, a.gated, kind, hh);
  // every global load of this wave is issued here, before any use
  const uint32_t y2 = *reinterpret_cast<const uint32_t*>(a.qkv + (size_t)m * ncols + (size_t)h * hd + 2 * lane);
  // (unconditional: loads that a head kind does not need read valid memory
  // and are ignored, so no branch separates them from the others)
  const float* nwp = kind == 0 ? a.q_norm : (kind == 1 ? a.k_norm : nullptr);
  const float* nsrc = nwp ? nwp : a.rope_cos;
  const float nw0 = nsrc[2 * lane], nw1 = nsrc[2 * lane + 1];
  float cs_e[2], sn_e[2];
#pragma unroll
  for (int e2 = 0; e2 < 2; ++e2) {
    const int e = 2 * lane + e2;
    const int ix = e < half ? e : (e < 2 * half ? e - half : 0);
    cs_e[e2] = a.rope_cos[(size_t)pos * half + ix];
    sn_e[e2] = a.rope_sin[(size_t)pos * half + ix];
  }
  const int page = kv.block_table[(size_t)seq * kv.max_pages + pos / kv.page];
  const float r0 = ifrd::h2f((uint16_t)(y2 & 0xFFFF)), r1 = ifrd::h2f((uint16_t)(y2 >> 16));
  // q/k norm and RoPE are evaluated for every head (v heads select the raw
  // values at the end): no branch, so the loads above stay ahead of all uses.
  x[2 * lane] = r0;
  x[2 * lane + 1] = r1;
  ifrd::wave_sync();
  // RMSNorm(1+w) of the head: eight sequential fused chains (reference AVX2
  // order, main.cpp:306-351)
  if (lane < 8) {
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = x[lane + 8 * i];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = fmaf(t[i], t[i], acc);
    red[w][lane] = acc;
  }
  ifrd::wave_sync();
  const float s0 = red[w][0] + red[w][4], s1 = red[w][1] + red[w][5];
  const float s2 = red[w][2] + red[w][6], s3 = red[w][3] + red[w][7];
  const float tot = (s0 + s1) + (s2 + s3);
  const float f = 1.0f / sqrtf(tot / (float)hd + a.eps);
  float v0 = nwp ? (r0 * f) * (1.0f + nw0) : r0;
  float v1 = nwp ? (r1 * f) * (1.0f + nw1) : r1;
  ifrd::wave_sync();
  x[2 * lane] = v0;
  x[2 * lane + 1] = v1;
  ifrd::wave_sync();
  // rotate-half RoPE on the first `rotary` dims (main.cpp:365-373)
  float o[2] = {v0, v1};
#pragma unroll
  for (int e2 = 0; e2 < 2; ++e2) {
    const int e = 2 * lane + e2;
    const int d = e < half ? e : e - half;
    const float xa = x[d], xb = x[min(d + half, hd - 1)];
    if (e < half) {
      o[e2] = xa * cs_e[e2] - xb * sn_e[e2];
    } else if (e < 2 * half) {
      o[e2] = xa * sn_e[e2] + xb * cs_e[e2];
    }
  }
  v0 = kind < 2 ? o[0] : r0;
  v1 = kind < 2 ? o[1] : r1;
  v0 = ifrd::fp16r(v0);
  v1 = ifrd::fp16r(v1);
  if (kind == 0 || kind == 3) {  // q after norm + RoPE; the gate as computed
    uint16_t* dst = (kind == 0 ? a.qout : a.gout) + ((size_t)m * nq + hh) * hd;
    *reinterpret_cast<uint32_t*>(dst + 2 * lane) = (uint32_t)ifrd::f2h(v0) | ((uint32_t)ifrd::f2h(v1) << 16);
    return;
  }
  const int tok = pos % kv.page;
  const size_t base = ((size_t)page * nkv + hh);
  if (!kv.kv_int8) {
    if (kind == 1) {  // dims 2l, 2l + 1 are adjacent elements of one K fragment lane
      uint16_t* kp = reinterpret_cast<uint16_t*>(kv.kpool) + base * kv.page * hd;
      *reinterpret_cast<uint32_t*>(kp + kv_koff(tok, 2 * lane)) =
          (uint32_t)ifrd::f2h(v0) | ((uint32_t)ifrd::f2h(v1) << 16);
    } else {
      uint16_t* vp = reinterpret_cast<uint16_t*>(kv.vpool) + base * hd * kv.page;
      vp[kv_voff(tok, 2 * lane)] = ifrd::f2h(v0);
      vp[kv_voff(tok, 2 * lane + 1)] = ifrd::f2h(v1);
    }
  } else {
    const float mx = ifrd::wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const uint16_t sh16 = ifrd::f2h(mx > 0.0f ? mx / 127.0f : 1.0f);
    const float s = ifrd::h2f(sh16);
    const float inv = 1.0f / s;
    const float t0 = v0 * inv, t1 = v1 * inv;
    int q0 = (int)(t0 >= 0.0f ? t0 + 0.5f : t0 - 0.5f);
    int q1 = (int)(t1 >= 0.0f ? t1 + 0.5f : t1 - 0.5f);
    q0 = min(127, max(-127, q0));
    q1 = min(127, max(-127, q1));
    if (kind == 1) {
      int8_t* kp = reinterpret_cast<int8_t*>(kv.kpool) + base * kv.page * hd;
      kp[kv_koff(tok, 2 * lane)] = (int8_t)q0;
      kp[kv_koff(tok, 2 * lane + 1)] = (int8_t)q1;
      if (lane == 0) kv.kscale[base * kv.page + tok] = sh16;
    } else {
      int8_t* vp = reinterpret_cast<int8_t*>(kv.vpool) + base * hd * kv.page;
      vp[kv_voff(tok, 2 * lane)] = (int8_t)q0;
      vp[kv_voff(tok, 2 * lane + 1)] = (int8_t)q1;
      if (lane == 0) kv.vscale[base * kv.page + tok] = sh16;
    }
  }
}

// ---- ragged batch packing ------------------------------------------------------
// Inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane
// row with DPP row_shr (lanes shifted in from outside the row read 0), then
// the three lower rows' totals added from scalars.  No LDS crossbar.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += ifrd::dpp_i<0x111>(x);  // row_shr:1
  x += ifrd::dpp_i<0x112>(x);  // row_shr:2
  x += ifrd::dpp_i<0x114>(x);  // row_shr:4
  x += ifrd::dpp_i<0x118>(x);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
            r2 = __builtin_amdgcn_readlane(x, 47);
  const int lane = threadIdx.x & 63;
  return x + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

// Block-wide exclusive scans of NA arrays v[a][0..n) in LDS, one pass;
// returns the totals.  Each thread takes a contiguous chunk of elements and
// gets their values from f(i, x) (x[a] = element i of array a; f runs in the
// thread that owns i, before any barrier), sums them, the chunk sums are
// scanned per wave, and every wave then scans the 16 wave totals itself (one
// LDS exchange, two barriers).  On return v[a][i] holds the prefix before i,
// and v[a][n] the total where total_at_n.  tmp holds NA (blockDim / 64) ints.
// E: int, or uint16_t for arrays whose prefixes stay below 65536.
template <int NA>
struct ScanTotals {
  int t[NA];
};
template <int NA, typename E, typename F>
__device__ ScanTotals<NA> block_exscan_f(E* const (&v)[NA], int n, bool total_at_n, int* tmp, F f) {
  const int T = blockDim.x, lane = threadIdx.x & 63, nw = T >> 6;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per = (n + T - 1) / T;
  const int b = threadIdx.x * per, e = min(n, b + per);
  int s[NA], incl[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) s[a] = 0;
  for (int i = b; i < e; ++i) {
    int x[NA];
    f(i, x);
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      v[a][i] = (E)x[a];
      s[a] += x[a];
    }
  }
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    incl[a] = wave_incl_scan(s[a]);
    if (lane == 63) tmp[a * nw + w] = incl[a];
  }
  __syncthreads();
  ScanTotals<NA> tot;
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    const int ws = wave_incl_scan(lane < nw ? tmp[a * nw + lane] : 0);
    const int before = w > 0 ? __builtin_amdgcn_readlane(ws, w - 1) : 0;
    tot.t[a] = __builtin_amdgcn_readlane(ws, nw - 1);
    int run = before + incl[a] - s[a];
    for (int i = b; i < e; ++i) {  // this thread's own elements: no barrier needed
      const int x = v[a][i];
      v[a][i] = (E)run;
      run += x;
    }
    if (total_at_n && threadIdx.x == 0) v[a][n] = (E)tot.t[a];
  }
  __syncthreads();
  return tot;
}

// The group of q-block t: the last g < ngroups with nblk[g] <= t.
__device__ __forceinline__ int pack_group_of(const uint16_t* nblk, int ngroups, int t) {
  int lo = 0, hi = ngroups - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (nblk[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// kPackGroups workgroups of kPackThreads.  Each builds the whole set of maps
// in its own LDS (the batch is at most 6144 rows), and the workgroups share
// the writes: workgroup g stores the per-row outputs of the rows its wave g
// holds, and every kPackGroups-th (q-block, kv head) pair's units and
// dispatch slots.  Row m = threadIdx.x + k kPackThreads is read from global
// memory once, into registers (k < kPackRowsPerThread); every later phase
// works from those registers and six LDS arrays, and every loop runs over
// rows, groups or q-blocks in parallel (no thread walks a group's q-blocks
// or quads).  Ten barriers in all.  LDS arrays, one map per phase (the
// three index maps, all <= 6144, in 16 bits: 159.9 KB at M = 6144):
//   fs, fw  group-start / want flags of row m (scanned: starts / wants before
//           m), then the per-q-block dispatch-slot counts (scanned)
//   gpos    first KV position of group g
//   gseq    sequence of group g
//   ucnt    first unit of q-block b
//   g0      first row of group g (M at ngroups)         16 bits
//   nblk    first q-block of group g (nb at ngroups)    16 bits
//   bgrp    group of q-block b                          16 bits
constexpr int kPackThreads = 1024, kPackRowsPerThread = 6, kPackMaxRows = kPackThreads * kPackRowsPerThread;
constexpr int kPackGroups = 16;
static_assert(kPackMaxRows < 65536, "the 16-bit index maps hold row, group and q-block indices");

__global__ __launch_bounds__(kPackThreads) void pack_kernel(const int32_t* rows, int M, int nkv, int qb,
                                                            int split, PackOut o) {
  extern __shared__ int sm[];
  int* fs = sm;                  // [M]
  int* fw = sm + M;              // [M]
  int* gpos = sm + 2 * M;        // [M]
  int* gseq = sm + 3 * M;        // [M]
  int* ucnt = sm + 4 * M;        // [M]
  int* tmp = sm + 5 * M;         // [2 kPackThreads / 64]
  uint16_t* g0 = reinterpret_cast<uint16_t*>(tmp + 2 * kPackThreads / 64);  // [M + 1]
  uint16_t* nblk = g0 + M + 1;   // [M + 1]
  uint16_t* bgrp = nblk + M + 1; // [M]
  constexpr int R = kPackRowsPerThread;
  // this workgroup's share of the writes: pairs t0, t0 + tstep, ... (64
  // consecutive pairs per wave: a store instruction costs about the same
  // whether 4 or 64 of its lanes are active); the rows of wave wg
  const int wg = blockIdx.x, t0 = wg + kPackGroups * threadIdx.x, tstep = kPackGroups * kPackThreads;
  const bool rows_out = (int)(threadIdx.x >> 6) == wg;
  // KV splits of a q-block of group g ending at its block b (q-block rows up to (b + 1) qb)
  auto nsplit = [&](int g, int b) {
    return (gpos[g] + min((b + 1) * qb, g0[g + 1] - g0[g]) + split - 1) / split;
  };
  int seq_r[R], pos_r[R], g_r[R];
  bool start_r[R], want_r[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int m = threadIdx.x + k * kPackThreads;
    start_r[k] = want_r[k] = false;
    seq_r[k] = pos_r[k] = g_r[k] = 0;
    if (m < M) {
      const int32_t* r = rows + 5 * m;
      const int seq = r[0], pos = r[1], tok = r[2], kind = r[3], want = r[4];
      const bool st = m == 0 || rows[5 * (m - 1)] != seq;
      seq_r[k] = seq;
      pos_r[k] = pos;
      start_r[k] = st;
      want_r[k] = want != 0;
      fs[m] = st ? 1 : 0;
      fw[m] = want ? 1 : 0;
      if (rows_out) {
        o.row_seq[m] = seq;
        o.row_pos[m] = pos;
        o.row_kind[m] = kind;
        if (o.row_tok) o.row_tok[m] = tok;
      }
    }
  }
  __syncthreads();
  int* const sflags[2] = {fs, fw};
  const int ngroups = block_exscan_f<2, int>(sflags, M, false, tmp, [&](int i, int (&x)[2]) {
    x[0] = fs[i];
    x[1] = fw[i];
  }).t[0];
  // each row: its group and the wanted-row list; group starts: first row,
  // position and sequence of each group
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int m = threadIdx.x + k * kPackThreads;
    if (m < M) {
      const int g = fs[m] + (start_r[k] ? 1 : 0) - 1;
      g_r[k] = g;
      if (rows_out) {
        o.row_grp[m] = g;
        if (want_r[k]) o.want_rows[fw[m]] = m;
      }
      if (start_r[k]) {
        g0[g] = (uint16_t)m;
        gpos[g] = pos_r[k];
        gseq[g] = seq_r[k];
      }
    }
  }
  if (threadIdx.x == 0) g0[ngroups] = (uint16_t)M;
  __syncthreads();
  if (wg == 0)
    for (int g = threadIdx.x; g <= ngroups; g += kPackThreads) o.cu_seqlens[g] = g0[g];
  uint16_t* const sblk[1] = {nblk};
  const int nb = block_exscan_f<1, uint16_t>(sblk, ngroups, true, tmp, [&](int g, int (&x)[1]) {
    x[0] = (g0[g + 1] - g0[g] + qb - 1) / qb;  // q-blocks of group g
  }).t[0];
  int* const sunits[1] = {ucnt};
  block_exscan_f<1, int>(sunits, nb, false, tmp, [&](int t, int (&x)[1]) {
    const int g = pack_group_of(nblk, ngroups, t);
    bgrp[t] = (uint16_t)g;
    x[0] = nkv * nsplit(g, t - nblk[g]);  // units of q-block t
  });
  // one thread per (q-block, kv head): that head's units of the q-block
  for (int t = t0; t < nb * nkv; t += tstep) {
    const int gb = t / nkv, kvh = t - gb * nkv;
    const int g = bgrp[gb], b = gb - nblk[g];
    const int r0 = g0[g], len = g0[g + 1] - r0, pos0 = gpos[g], seq = gseq[g];
    const int qn = min(qb, len - b * qb);
    const int kvhi = pos0 + b * qb + qn;
    const int ns = (kvhi + split - 1) / split;
    const int base = ucnt[gb];
    for (int s = 0; s < ns; ++s) {
      AttnUnit u;
      u.seq = seq;
      u.kvh = kvh;
      u.row0 = r0 + b * qb;
      u.qn = qn;
      u.qpos0 = pos0 + b * qb;
      u.kv_lo = s * split;
      u.kv_hi = min((s + 1) * split, kvhi);
      u.pad = 0;
      o.units[base + kvh * ns + s] = u;
    }
  }
  // each row's combine map (q-block gb = its group's first block + (m - r0) / qb)
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int m = threadIdx.x + k * kPackThreads;
    if (m < M && rows_out) {
      const int g = g_r[k], r0 = g0[g], len = g0[g + 1] - r0, pos0 = gpos[g];
      const int b = (m - r0) / qb, gb = nblk[g] + b;
      const int qn = min(qb, len - b * qb);
      o.comb_base[m] = ucnt[gb];
      o.comb_nsplit[m] = (pos0 + b * qb + qn + split - 1) / split;
      o.comb_tok[m] = m - r0 - b * qb;
    }
  }
  // ---- dispatch order (see attn_slot_count), counts per q-block in q-block
  // order.  Chunked region (fs): a group of several q-blocks is cut into
  // quads of 4 consecutive q-blocks, each quad taking 4 nkv slots per KV
  // split of its last q-block, counted at that q-block.  Dense region after
  // it (fw): groups of one q-block, their units packed in unit order.
  int* const sslots[2] = {fs, fw};
  const int CS = block_exscan_f<2, int>(sslots, nb, false, tmp, [&](int t, int (&x)[2]) {
    const int g = bgrp[t], nbg = nblk[g + 1] - nblk[g], b = t - nblk[g];
    x[0] = (nbg > 1 && ((b & 3) == 3 || b == nbg - 1)) ? 4 * nkv * nsplit(g, b) : 0;
    x[1] = nbg == 1 ? nkv * nsplit(g, 0) : 0;
  }).t[0];
  // one thread per (q-block, kv head): that head's slots of the q-block
  for (int t = t0; t < nb * nkv; t += tstep) {
    const int gb = t / nkv, kvh = t - gb * nkv;
    const int g = bgrp[gb], nbg = nblk[g + 1] - nblk[g], b = gb - nblk[g];
    const int ns = nsplit(g, b), base = ucnt[gb];
    if (nbg == 1) {
      for (int s = 0; s < ns; ++s) o.order[CS + fw[gb] + kvh * ns + s] = base + kvh * ns + s;
      continue;
    }
    const int q = b & 3, bl = min((b | 3), nbg - 1);  // the quad's last q-block
    const int off = fs[nblk[g] + bl], nsm = nsplit(g, bl);
    for (int s = 0; s < nsm; ++s) o.order[off + (kvh * nsm + s) * 4 + q] = s < ns ? base + kvh * ns + s : -1;
    // slots of absent q-blocks in a short last quad
    if (b == nbg - 1)
      for (int qq = q + 1; qq < 4; ++qq)
        for (int s = 0; s < nsm; ++s) o.order[off + (kvh * nsm + s) * 4 + qq] = -1;
  }
}

}  // namespace

long attn_slot_count(const int* g_pos0, const int* g_len, int ngroups, int nkv, int split, int qb,
                     long* chunked) {
  long dense = 0, chunk = 0;
  for (int g = 0; g < ngroups; ++g) {
    const int nbg = (g_len[g] + qb - 1) / qb;
    if (nbg == 1) {
      dense += (long)nkv * ((g_pos0[g] + g_len[g] + split - 1) / split);
      continue;
    }
    for (int j = 0; 4 * j < nbg; ++j) {
      const int bl = std::min(4 * j + 3, nbg - 1);
      chunk += 4L * nkv * ((g_pos0[g] + std::min((bl + 1) * qb, g_len[g]) + split - 1) / split);
    }
  }
  if (chunked) *chunked = chunk;
  return chunk + dense;
}

namespace {

// mg = fp16(silu(g) * u) over an unpaired [M][2F] gate|up buffer (used when
// gate and up have different bit widths and cannot share one launch).
__global__ void swiglu_kernel(const uint16_t* gu, int F, uint16_t* mg) {
  const int m = blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < F; i += gridDim.x * blockDim.x) {
    const float g = ifrd::h2f(gu[(size_t)m * 2 * F + i]);
    const float u = ifrd::h2f(gu[(size_t)m * 2 * F + F + i]);
    mg[(size_t)m * F + i] = ifrd::f2h(g / (1.0f + expf(-g)) * u);
  }
}

__global__ void gather_rows_kernel(const float* src, const int32_t* rows, int H, float* dst) {
  const int i = blockIdx.x;
  const float* s = src + (size_t)rows[i] * H;
  for (int k = threadIdx.x; k < H; k += blockDim.x) dst[(size_t)i * H + k] = s[k];
}

}  // namespace

// The generic row kernels stage a row in LDS; rows past 64 KB (K > 8000
// floats of staging) need the 160 KB dynamic-LDS limit, set once per kernel.
template <typename F>
hipError_t allow_big_lds(F* f, bool& done) {
  if (done) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(f),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (e == hipSuccess) done = true;
  return e;
}

namespace {

// grid (n pages, npools): one workgroup copies one page of one pool.
__global__ __launch_bounds__(256) void copy_pages_kernel(PageCopyArgs a) {
  const int i = blockIdx.x, j = blockIdx.y;
  const size_t words = a.page_bytes[j % a.per] / 16;
  const uint4* src = reinterpret_cast<const uint4*>(a.pools[j]) + (size_t)a.sp[i] * words;
  uint4* dst = reinterpret_cast<uint4*>(a.pools[j]) + (size_t)a.dp[i] * words;
  for (size_t w = threadIdx.x; w < words; w += blockDim.x) dst[w] = src[w];
}

}  // namespace

hipError_t launch_copy_pages(const PageCopyArgs& a, hipStream_t st) {
  if (a.n <= 0) return hipSuccess;
  if (!a.pools || !a.sp || !a.dp || a.npools <= 0 || a.per < 1 || a.per > 4 || a.npools % a.per != 0)
    return hipErrorInvalidValue;
  for (int k = 0; k < a.per; ++k)
    if (a.page_bytes[k] == 0 || a.page_bytes[k] % 16 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(copy_pages_kernel, dim3(a.n, a.npools), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_row_quant(const RowQuantArgs& a, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (a.K <= 0 || a.K % 128 != 0 || a.K > 8192 || !a.q || !a.qscale) return hipErrorInvalidValue;
  if (a.ga != 0 && (a.ga != 64 || a.K / 64 > 192)) return hipErrorInvalidValue;
  if (a.src == SRC_X && !a.x) return hipErrorInvalidValue;
  if (a.src == SRC_EMBED && (!a.embed || !a.tokens || !a.resid)) return hipErrorInvalidValue;
  if (a.src == SRC_RESID && (!a.y || !a.resid)) return hipErrorInvalidValue;
  if (a.K == 1024 && (a.ga == 0 || a.ga == 64)) {
    hipLaunchKernelGGL(row_quant1024_kernel, dim3(a.M), dim3(512), 0, st, a);
    return hipGetLastError();
  }
  {
    // the register kernel: K a multiple of 256, head P = floor_pow2(K) and a
    // tail (K - P) / 256 per thread that is 0 or a power of two
    int P = 256;
    while (2 * P <= a.K) P *= 2;
    const int et = (a.K - P) / 256;
    if (a.K % 256 == 0 && (et & (et - 1)) == 0) {
      switch (P / 256) {
        case 1: hipLaunchKernelGGL(row_quant_wide<1>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        case 2: hipLaunchKernelGGL(row_quant_wide<2>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        case 4: hipLaunchKernelGGL(row_quant_wide<4>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        case 8: hipLaunchKernelGGL(row_quant_wide<8>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        case 16: hipLaunchKernelGGL(row_quant_wide<16>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        case 32: hipLaunchKernelGGL(row_quant_wide<32>, dim3(a.M), dim3(256), 0, st, a); return hipGetLastError();
        default: break;
      }
    }
  }
  const size_t lds = (size_t)(2 * a.K + 64 + a.K / 64) * sizeof(float);
  static bool big = false;
  if (hipError_t e = allow_big_lds(row_quant_kernel, big)) return e;
  hipLaunchKernelGGL(row_quant_kernel, dim3(a.M), dim3(256), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_quant_plain(const float* xf, const uint16_t* xh, int M, int K, int8_t* q,
                              float* qscale, float* gsum, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || K % 128 != 0 || K > kQuantPlainMaxK || (!xf && !xh) || !q || !qscale)
    return hipErrorInvalidValue;
  if (K == 2048) {
    hipLaunchKernelGGL(quant_plain8<256>, dim3(M), dim3(256), 0, st, xf, xh, q, qscale, gsum);
    return hipGetLastError();
  }
  if (K == 3072) {
    hipLaunchKernelGGL(quant_plain8<384>, dim3(M), dim3(384), 0, st, xf, xh, q, qscale, gsum);
    return hipGetLastError();
  }
  if (K == 4096) {
    hipLaunchKernelGGL(quant_plain8<512>, dim3(M), dim3(512), 0, st, xf, xh, q, qscale, gsum);
    return hipGetLastError();
  }
  switch ((K + 2047) / 2048) {
#define IFR_QPW(CH)                                                                         \
  case CH:                                                                                   \
    hipLaunchKernelGGL(quant_plain_wide<CH>, dim3(M), dim3(256), 0, st, xf, xh, K, q, qscale, gsum); \
    break;
    IFR_QPW(1) IFR_QPW(2) IFR_QPW(3) IFR_QPW(4) IFR_QPW(5)
    IFR_QPW(6) IFR_QPW(7) IFR_QPW(8) IFR_QPW(9) IFR_QPW(10)
#undef IFR_QPW
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_qk_rope_kv(const QKArgs& a, const KVLayout& kv, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (kv.hd != 128 || a.rotary <= 0 || a.rotary > kv.hd || a.rotary % 2 != 0 || kv.page <= 0 ||
      !a.qkv || !a.qout || !kv.kpool || !kv.vpool || !kv.block_table || (a.gated && !a.gout))
    return hipErrorInvalidValue;
  if (kv.kv_int8 && (!kv.kscale || !kv.vscale)) return hipErrorInvalidValue;
  const int heads = (a.gated ? 2 * a.nq : a.nq) + 2 * kv.nkv;
  hipLaunchKernelGGL(qk_rope_kv_kernel, dim3(a.M, (heads + 3) / 4), dim3(256), 0, st, a, kv);
  return hipGetLastError();
}

hipError_t launch_pack(const int32_t* rows, int M, int nkv, int qb, int split, const PackOut& o,
                       hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (M > kPackMaxRows || qb <= 0 || split <= 0 || nkv <= 0) return hipErrorInvalidValue;
  const size_t lds = (size_t)(5 * M + 2 * kPackThreads / 64) * sizeof(int) + (size_t)(3 * M + 2) * sizeof(uint16_t);
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(pack_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hipLaunchKernelGGL(pack_kernel, dim3(kPackGroups), dim3(kPackThreads), lds, st, rows, M, nkv, qb, split, o);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* gu, int M, int F, uint16_t* mg, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((F + 255) / 256, M), dim3(256), 0, st, gu, F, mg);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const float* src, const int32_t* rows, int n, int H, float* dst,
                              hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(n), dim3(256), 0, st, src, rows, H, dst);
  return hipGetLastError();
}

}  // namespace ifrk
