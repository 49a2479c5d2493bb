// W2A8 / W4A8 / W8A8 quantized GEMM on gfx950 int8 MFMA with int32 accumulation.
//
// Integer contract (the W2A8 DPAS contract of the reference, dpas48_tiled,
// src/gemm/quant_gemm.cpp:3602-3736, generalized to per-(row,group) scale and
// zero):  for each 128-wide K group g
//     T(m,n,g) = sum_k a_q(m,k) * code(n,k)      exact int32, v_mfma_i32_16x16x64_i8
//     S(m,g)   = sum_k a_q(m,k)                  from the activation producer
//     d   = fma(-zero(n,g), S, T)
//     acc = fma(scale(n,g), d, acc)              groups strictly ascending
// y(m,n) = fp16_rne((ascale(m) * post) * acc), post a per-linear fp32 factor
// (1 leaves ascale unchanged).  The fold order is fixed per output
// element: split-K variants exchange the int32 T through LDS and fold them in
// group order, so every launch shape produces the same bits.
//
// Codebook linears (every zero(n,g) = C/2, C = 2^bits - 1: the reference's
// canonical codebook, dashq.cpp:405-417) take a two-operation fold with the
// same bits.  The MFMA runs over the doubled codes 2c and starts each group's
// accumulator at the integer 0x4B400000, whose bits read as the float
// 1.5 * 2^23: the accumulator's bits then read as the float 1.5 * 2^23 + 2T
// exactly (|2T| < 2^22).  With Y(m,g) = 1.5 * 2^23 + C * S(m,g) (an exact
// integer below 2^24) and h(n,g) = scale(n,g) / 2 (exact),
//     d2  = T_float - Y          = 2T - C S = 2 (T - zero S)   exact
//     acc = fma(h, d2, acc)
// and fma(h, d2, acc) == fma(scale, d, acc) because both products are the
// same real number and d = fma(-zero, S, T) is exact for these codes (a
// multiple of 1/2 below 2^20).  No int->float conversion, one subtract.
//
// Tiling: a workgroup is 4 waves (256 lanes).  Each wave owns WM x WN tiles of
// 16x16 outputs (MFMA 16x16x64).  The fold-side operands (S, scale/zero) are
// staged in LDS once per workgroup so the K loop carries only the A and B
// fragment loads.  qgemm_rows (larger M): each wave folds its own
// accumulators while the next R groups are in flight in registers.
// qgemm_splitk (M <= 64, the weight-stream-bound decode shapes): the 4 waves
// split the K groups of one tile block and fold after one LDS exchange.  Codes
// are read in the fragment-major layout, one fully coalesced 256*bits/8-byte
// block per (tile, K step).
#include "ifr_dev.h"
#include "ifr_kernels.h"

#include <algorithm>
#include <thread>
#include <vector>

namespace ifrk {
namespace qg {

constexpr int kG = 128;
// groups in flight per wave in the decode weight stream's ring
constexpr int kStreamRing = 4;

struct KParams {
  const int8_t* a;
  const float* as;
  const float* gs;
  const uint32_t* codes;
  const uint32_t* sz;
  uint16_t* out;
  int32_t* tdump;
  int M, N, K, ng, nsteps, ldo;
  float post;  // folded into the row scale: (ascale * post) * acc
  // qgemm_rows block order.  swz > 0: a 1-D grid in which the blocks of
  // each XCD (block id mod 8) own the column blocks of that residue and walk
  // all row blocks over swz of them at a time, so the weight columns in
  // flight on an XCD stay inside its L2.  swz < 0: the same with the roles
  // of rows and columns exchanged (activation rows kept, for a larger A).
  // The owned dimension is padded to a multiple of 8; padding blocks exit.
  int nbx, nby, swz;
  // 1: every zero of the linear is C/2 (the codebook fold applies)
  int ff;
  // 1: out is 16-byte aligned and ldo a multiple of 8, so qgemm_rows stores
  // its output tile as 16-byte row chunks
  int vst;
  // qgemm_stream: the pitch (in groups) of its parked d and scale rows
  int spitch;
  // EPI 2 (QKV projection with the q/k norm + RoPE + KV append epilogue):
  // the arguments of the separate pass (row maps, norms, RoPE tables, q
  // output, paged KV)
  QKArgs qa;
  KVLayout kv;
  // optional: the codes of A row-major [M][K] (the weight stream stages its
  // A rows from here when given)
  const int8_t* arow;
};

// One compilation of this file per code width (IFR_QGEMM_BITS = 2, 4, 8)
// instantiates that width's kernels; the build without it holds the packing
// and the dispatch.
hipError_t launch_b2(const KParams& p, int epi, int variant, hipStream_t st);
hipError_t launch_b4(const KParams& p, int epi, int variant, hipStream_t st);
hipError_t launch_b8(const KParams& p, int epi, int variant, hipStream_t st);

}  // namespace qg

#if defined(IFR_QGEMM_BITS)
namespace qg {
namespace {


// Raw code dwords of one lane for one K step, and their unpacking into the
// int8 B operand: operand dword d holds codes j = 4d..4d+3 in bytes 0..3
// (INT2: byte b of dword d is bits [8b + 2d, +2) of the packed dword; INT4:
// bits [8b + 4(d%2), +4) of packed dword d/2; INT8: stored directly).
template <int BITS>
__device__ __forceinline__ void load_raw(const uint32_t* __restrict__ base, int lane,
                                         uint32_t (&w)[BITS / 2]) {
  if constexpr (BITS == 2) {
    w[0] = __builtin_nontemporal_load(base + lane);
  } else if constexpr (BITS == 4) {
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    const v2u x = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(base) + lane);
    w[0] = x.x;
    w[1] = x.y;
  } else {
    const v4i x = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(base) + lane);
    w[0] = (uint32_t)x.x;
    w[1] = (uint32_t)x.y;
    w[2] = (uint32_t)x.z;
    w[3] = (uint32_t)x.w;
  }
}
template <int BITS, bool DBL = false>
__device__ __forceinline__ v4i unpack_b(const uint32_t (&w)[BITS / 2]) {
  v4i r;
  if constexpr (DBL && BITS == 2) {  // 2c: the same fields, one bit higher
    r.x = (int)((w[0] << 1) & 0x06060606u);
    r.y = (int)((w[0] >> 1) & 0x06060606u);
    r.z = (int)((w[0] >> 3) & 0x06060606u);
    r.w = (int)((w[0] >> 5) & 0x06060606u);
  } else if constexpr (DBL && BITS == 4) {
    r.x = (int)((w[0] << 1) & 0x1E1E1E1Eu);
    r.y = (int)((w[0] >> 3) & 0x1E1E1E1Eu);
    r.z = (int)((w[1] << 1) & 0x1E1E1E1Eu);
    r.w = (int)((w[1] >> 3) & 0x1E1E1E1Eu);
  } else if constexpr (BITS == 2) {
    r.x = (int)(w[0] & 0x03030303u);
    r.y = (int)((w[0] >> 2) & 0x03030303u);
    r.z = (int)((w[0] >> 4) & 0x03030303u);
    r.w = (int)((w[0] >> 6) & 0x03030303u);
  } else if constexpr (BITS == 4) {
    r.x = (int)(w[0] & 0x0F0F0F0Fu);
    r.y = (int)((w[0] >> 4) & 0x0F0F0F0Fu);
    r.z = (int)(w[1] & 0x0F0F0F0Fu);
    r.w = (int)((w[1] >> 4) & 0x0F0F0F0Fu);
  } else {
    r.x = (int)w[0];
    r.y = (int)w[1];
    r.z = (int)w[2];
    r.w = (int)w[3];
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


__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ void store_plain(const KParams& p, int row, int col, float as, float acc) {
  p.out[(size_t)row * p.ldo + col] = ifrd::f2h(as * acc);
}
__device__ __forceinline__ void store_swiglu(const KParams& p, int row, int col, float as, float accg,
                                             float accu) {
  const float g = ifrd::fp16r(as * accg);
  const float u = ifrd::fp16r(as * accu);
  p.out[(size_t)row * p.ldo + col] = ifrd::f2h(silu_f(g) * u);
}

// Operands of one 128-wide K group (two MFMA K steps) of one wave.
template <int BITS, int WM, int WN>
struct GroupOps {
  v4i A[2][WM];
  uint32_t B[2][WN][BITS / 2];
};

// A: tile offsets aoff[i] (bytes, per lane) from the uniform base p.a, one
// contiguous 1 KB A tile per (16 rows, K step);
// B: tile indices tl[j] are wave-uniform, so each (tile, step) block base is a
// scalar and the lane adds lane * bits/2 dwords.
template <int BITS, int WM, int WN>
__device__ __forceinline__ void load_ops(const KParams& p, const uint32_t (&aoff)[WM],
                                         const int (&tl)[WN], int lane, int g,
                                         GroupOps<BITS, WM, WN>& b) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = 2 * g + h;
    const int8_t* ab = p.a + 1024 * s;
#pragma unroll
    for (int i = 0; i < WM; ++i) b.A[h][i] = *reinterpret_cast<const v4i*>(ab + aoff[i]);
#pragma unroll
    for (int j = 0; j < WN; ++j)
      load_raw<BITS>(p.codes + ((size_t)tl[j] * p.nsteps + s) * 64 * (BITS / 2), lane, b.B[h][j]);
  }
}

// The bits of the float 1.5 * 2^23 (the codebook fold's accumulator start).
constexpr int kFoldBias = 0x4B400000;
constexpr float kFoldBiasF = 12582912.0f;

template <int BITS, int WM, int WN, bool FF = false>
__device__ __forceinline__ void mma_group(const GroupOps<BITS, WM, WN>& b, v4i (&T)[WM][WN]) {
  constexpr int c0 = FF ? kFoldBias : 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    v4i B[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) B[j] = unpack_b<BITS, FF>(b.B[h][j]);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
        T[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b.A[h][i], B[j], h ? T[i][j] : (v4i){c0, c0, c0, c0},
                                                        0, 0, 0);
  }
}

// Everything the fold needs besides T, staged in LDS once per workgroup:
// S_l[g][BM] (group code sums of the block's rows) and Z_l[g][BN] (packed
// fp16 scale | zero << 16 of the block's columns).  Rows past M read row M-1
// and columns past N read the last tile; their outputs are never stored.
// Up to NQ elements per thread are fetched with all loads in flight at once;
// larger blocks (K > 128 * NQ * 256 / max(BM, BN)) take a plain loop.
// FF (codebook fold): S_l holds Y = 1.5 * 2^23 + C * S and Z_l the fp32
// scale / 2 instead (see the header).
template <int BM, int BN, int NQ, int BITS = 2, bool FF = false>
__device__ __forceinline__ void stage_fold_operands(const KParams& p, int bm0, int bt0, float* S_l,
                                                    uint32_t* Z_l) {
  constexpr float C = (float)((1 << BITS) - 1);
  auto sval = [&](float sv) { return FF ? kFoldBiasF + C * sv : sv; };
  auto zval = [&](uint32_t zw) {
    return FF ? __float_as_uint(0.5f * ifrd::h2f((uint16_t)(zw & 0xFFFFu))) : zw;
  };
  const int ng = p.ng, ntiles = p.N >> 4;
  constexpr int TB = BN / 16;
  auto s_src = [&](int t) {  // t = g * BM + r
    return p.gs + (size_t)min(bm0 + (t % BM), p.M - 1) * ng + t / BM;
  };
  auto z_src = [&](int t) {  // t = (g * TB + jt) * 16 + c
    const int c = t & 15, jt = (t >> 4) % TB, g = (t >> 4) / TB;
    return p.sz + ((size_t)min(bt0 + jt, ntiles - 1) * ng + g) * 16 + c;
  };
  auto z_dst = [&](int t) {
    const int c = t & 15, jt = (t >> 4) % TB, g = (t >> 4) / TB;
    return g * BN + 16 * jt + c;
  };
  if (BM * ng <= 256 * NQ && BN * ng <= 256 * NQ) {
    float sv[NQ];
    uint32_t zv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + 256 * q;
      if (t < BM * ng) sv[q] = *s_src(t);
      if (t < BN * ng) zv[q] = *z_src(t);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + 256 * q;
      if (t < BM * ng) S_l[t] = sval(sv[q]);
      if (t < BN * ng) Z_l[z_dst(t)] = zval(zv[q]);
    }
  } else {
    for (int t = threadIdx.x; t < BM * ng; t += 256) S_l[t] = sval(*s_src(t));
    for (int t = threadIdx.x; t < BN * ng; t += 256) Z_l[z_dst(t)] = zval(*z_src(t));
  }
}

// ---- QKV epilogue: q/k RMSNorm(1 + w) + RoPE + KV append ----------------------
// For a block of BM rows x one 128-column head (BN = 128): the fp16-rounded
// outputs y = fp16(ascale * post * acc) -- the values the separate
// qk_rope_kv_kernel reads back -- are staged in LDS, then each wave takes 8
// rows with 8 lanes per row.  Lane s of a row owns dims 8 s .. 8 s + 7 and
// their rotate-half partners 64 + 8 s .. + 7, so RoPE needs no exchange; the
// RMS sum runs the reference's eight chains (chain s over dims s + 8 n), and
// every value is formed as in qk_rope_kv_kernel, so the results are
// bit-identical.  Requires hd = 128 and rotary = 128.
template <int BM, int BN, int WM, int WN, int MW>
__device__ __forceinline__ void qk_epilogue(const KParams& p, float* lds, const v4f (&acc)[WM][WN],
                                            const float (&asr)[WM][4], int bm0, int bt0, int wave, int lane) {
  static_assert(BN == 128 && BM == 32, "one 128-column head of 32 rows per workgroup");
  constexpr int NW = 4 / MW, YS = BN + 4;  // padded LDS row
  const QKArgs& qa = p.qa;
  const KVLayout& kv = p.kv;
  const int nq = qa.nq, nkv = kv.nkv;
  int kind, hh;  // q, k, v or gate
  qkv_block((bt0 * 16) / 128, nq, nkv, qa.gated, kind, hh);
  const int rr = lane >> 3, sub = lane & 7;
  const int row_l = 8 * wave + rr, m = bm0 + row_l;
  const int mc = min(m, p.M - 1);
  const int d0 = 8 * sub;
  // stage y (the fold-operand LDS is free once every wave has folded)
  float* Y = lds;
  float* red = lds + BM * YS;
  __syncthreads();
  {
    const int lrow = lane & 15, lgrp = lane >> 4;
    const int wm = wave % MW, wn = wave / MW;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          Y[(16 * WM * wm + 16 * i + 4 * lgrp + r) * YS + 16 * (WN * wn + j) + lrow] =
              ifrd::fp16r(asr[i][r] * acc[i][j][r]);
  }
  (void)NW;
  // then the row record, RoPE entries, norm weights and block table (issued
  // once the accumulators are dead, so they do not raise the register peak)
  const int pos = qa.row_pos[mc], seq = qa.row_seq[mc];
  float cs[8], sn[8], nwa[8], nwb[8];
  {
    const float4* cp = reinterpret_cast<const float4*>(qa.rope_cos + (size_t)pos * 64 + d0);
    const float4* sp = reinterpret_cast<const float4*>(qa.rope_sin + (size_t)pos * 64 + d0);
    // a model without q/k norm (or a v head) reads the RoPE table in its place
    // and ignores it, so the loads stay unconditional
    const float* nwh = kind == 0 ? qa.q_norm : (kind == 1 ? qa.k_norm : nullptr);
    const float* nw = nwh ? nwh : qa.rope_cos;
    const float4* na = reinterpret_cast<const float4*>(nw + d0);
    const float4* nb = reinterpret_cast<const float4*>(nw + 64 + d0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float4 c4 = cp[q], s4 = sp[q], a4 = na[q], b4 = nb[q];
      cs[4 * q] = c4.x; cs[4 * q + 1] = c4.y; cs[4 * q + 2] = c4.z; cs[4 * q + 3] = c4.w;
      sn[4 * q] = s4.x; sn[4 * q + 1] = s4.y; sn[4 * q + 2] = s4.z; sn[4 * q + 3] = s4.w;
      nwa[4 * q] = a4.x; nwa[4 * q + 1] = a4.y; nwa[4 * q + 2] = a4.z; nwa[4 * q + 3] = a4.w;
      nwb[4 * q] = b4.x; nwb[4 * q + 1] = b4.y; nwb[4 * q + 2] = b4.z; nwb[4 * q + 3] = b4.w;
    }
  }
  const bool has_norm = (kind == 0 ? qa.q_norm : qa.k_norm) != nullptr;
  const int page = kv.block_table[(size_t)seq * kv.max_pages + pos / kv.page];
  __syncthreads();
  if (m >= p.M) return;  // after the last workgroup barrier
  const float* y = Y + row_l * YS;
  float xa[8], xb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    xa[k] = y[d0 + k];
    xb[k] = y[64 + d0 + k];
  }
  // RMSNorm(1+w) of the head: chain `sub` over dims sub + 8 n (reference
  // AVX2 order, main.cpp:306-351)
  {
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = y[sub + 8 * i];
    float accn = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) accn = fmaf(t[i], t[i], accn);
    red[row_l * 8 + sub] = accn;
  }
  ifrd::wave_sync();
  const float* rd = red + row_l * 8;
  const float s0 = rd[0] + rd[4], s1 = rd[1] + rd[5];
  const float s2 = rd[2] + rd[6], s3 = rd[3] + rd[7];
  const float tot = (s0 + s1) + (s2 + s3);
  const float f = 1.0f / sqrtf(tot / 128.0f + qa.eps);
  float oa[8], ob[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (kind < 2) {
      // RMSNorm(1+w) only where the model has q/k norm weights (the separate
      // pass, qk_rope_kv_kernel, makes the same choice)
      const float va = has_norm ? (xa[k] * f) * (1.0f + nwa[k]) : xa[k];
      const float vb = has_norm ? (xb[k] * f) * (1.0f + nwb[k]) : xb[k];
      // rotate-half RoPE (main.cpp:365-373): dims d and d + 64 share entry d
      oa[k] = va * cs[k] - vb * sn[k];
      ob[k] = va * sn[k] + vb * cs[k];
    } else {
      oa[k] = xa[k];
      ob[k] = xb[k];
    }
    oa[k] = ifrd::fp16r(oa[k]);
    ob[k] = ifrd::fp16r(ob[k]);
  }
  auto pack8 = [&](const float (&v)[8]) {
    uint32_t w4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w4[k] = (uint32_t)ifrd::f2h(v[2 * k]) | ((uint32_t)ifrd::f2h(v[2 * k + 1]) << 16);
    return make_uint4(w4[0], w4[1], w4[2], w4[3]);
  };
  if (kind == 0 || kind == 3) {  // q after norm + RoPE; the gate as computed
    uint16_t* dst = (kind == 0 ? qa.qout : qa.gout) + ((size_t)m * nq + hh) * 128;
    *reinterpret_cast<uint4*>(dst + d0) = pack8(oa);
    *reinterpret_cast<uint4*>(dst + 64 + d0) = pack8(ob);
    return;
  }
  const int tok = pos % kv.page;
  const size_t base = (size_t)page * nkv + hh;
  if (!kv.kv_int8) {
    if (kind == 1) {  // 8 consecutive dims of one token are 16 contiguous bytes
      uint16_t* kp = reinterpret_cast<uint16_t*>(kv.kpool) + base * kv.page * 128;
      *reinterpret_cast<uint4*>(kp + kv_koff(tok, d0)) = pack8(oa);
      *reinterpret_cast<uint4*>(kp + kv_koff(tok, 64 + d0)) = pack8(ob);
    } else {
      uint16_t* vp = reinterpret_cast<uint16_t*>(kv.vpool) + base * 128 * kv.page;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        vp[kv_voff(tok, d0 + k)] = ifrd::f2h(oa[k]);
        vp[kv_voff(tok, 64 + d0 + k)] = ifrd::f2h(ob[k]);
      }
    }
  } else {
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fmaxf(fabsf(oa[k]), fabsf(ob[k])));
    // the row's 8 lanes: max is order-free
    mx = fmaxf(mx, ifrd::lane_xor<1>(mx));
    mx = fmaxf(mx, ifrd::lane_xor<2>(mx));
    mx = fmaxf(mx, ifrd::lane_xor<4>(mx));
    const uint16_t sh16 = ifrd::f2h(mx > 0.0f ? mx / 127.0f : 1.0f);
    const float sc = ifrd::h2f(sh16);
    const float inv = 1.0f / sc;
    auto code = [&](float v) {
      const float t = v * inv;
      int q = (int)(t >= 0.0f ? t + 0.5f : t - 0.5f);
      return (uint32_t)(min(127, max(-127, q)) & 0xFF);
    };
    if (kind == 1) {
      int8_t* kp = reinterpret_cast<int8_t*>(kv.kpool) + base * kv.page * 128;
      uint32_t la[2] = {0u, 0u}, lb[2] = {0u, 0u};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        la[k >> 2] |= code(oa[k]) << (8 * (k & 3));
        lb[k >> 2] |= code(ob[k]) << (8 * (k & 3));
      }
      *reinterpret_cast<uint2*>(kp + kv_koff(tok, d0)) = make_uint2(la[0], la[1]);
      *reinterpret_cast<uint2*>(kp + kv_koff(tok, 64 + d0)) = make_uint2(lb[0], lb[1]);
      if (sub == 0) kv.kscale[base * kv.page + tok] = sh16;
    } else {
      int8_t* vp = reinterpret_cast<int8_t*>(kv.vpool) + base * 128 * kv.page;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        vp[kv_voff(tok, d0 + k)] = (int8_t)code(oa[k]);
        vp[kv_voff(tok, 64 + d0 + k)] = (int8_t)code(ob[k]);
      }
      if (sub == 0) kv.vscale[base * kv.page + tok] = sh16;
    }
  }
}

// One K group's fold of a wave's WM x WN accumulators: S from the fold
// operand staged in LDS (S_l [ng][BM]), the packed fp16 scale | zero << 16
// of the lane's column of tile j in zr[j]: the general three-operation fold,
// or the codebook fold (FF: S_l holds Y, the scale is halved here); DUMP
// writes the true int32 T of every valid output.
template <int BITS, int WM, int WN, int MW, bool FF, bool DUMP>
__device__ __forceinline__ void fold_group(const KParams& p, const float* S_l, const uint32_t (&zr)[WN],
                                           const v4i (&T)[WM][WN], v4f (&acc)[WM][WN], int g, int wm, int wn,
                                           int lane, int row0, int tile0, const int (&tl)[WN]) {
  constexpr int BM = 16 * WM * MW;
  const int lrow = lane & 15, lgrp = lane >> 4;
  v4f S[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i)
    S[i] = *reinterpret_cast<const v4f*>(&S_l[g * BM + 16 * WM * wm + 16 * i + 4 * lgrp]);
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const uint32_t zw = zr[j];
    if constexpr (FF) {  // S holds Y; h = scale / 2 (exact)
      const float h = 0.5f * ifrd::h2f((uint16_t)(zw & 0xFFFFu));
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[i][j][r] = fmaf(h, __int_as_float(T[i][j][r]) - S[i][r], acc[i][j][r]);
      continue;
    }
    const float sc = ifrd::h2f((uint16_t)(zw & 0xFFFFu));
    const float ze = ifrd::h2f((uint16_t)(zw >> 16));
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t Tv = true_t<BITS>(T[i][j][r], S[i][r]);
        const float d = fmaf(-ze, S[i][r], (float)Tv);
        acc[i][j][r] = fmaf(sc, d, acc[i][j][r]);
        if (DUMP && row0 + 16 * i + 4 * lgrp + r < p.M && tile0 + j < (p.N >> 4))
          p.tdump[((size_t)(row0 + 16 * i + 4 * lgrp + r) * p.N + 16 * tl[j] + lrow) * p.ng + g] = Tv;
      }
  }
}

// The stores of one wave's WM x WN output tiles (EPI 0: plain, 1: the
// SwiGLU pair) of the whole-K kernel: the same code qgemm_rows has inline
// (called from there, the function raised the 27B gate/up launch from 168
// to 170 VGPRs, 3 -> 2 waves per SIMD, 45.3 -> 48.1 ms per cfg5 iteration).
// Every wave has read its last LDS operand before any wave passes the
// barrier of the 16-byte path.
template <int WM, int WN, int EPI, bool DUMP>
__device__ __forceinline__ void store_tiles(const KParams& p, float* lds_f, const v4f (&acc)[WM][WN],
                                            const float (&asr)[WM][4], int row0, int tile0, int wave,
                                            int lane) {
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.N >> 4;
  if (!DUMP && p.vst) {
    // The wave's output tile (16 WM rows x TC columns of fp16) is staged in
    // its own LDS slice and stored as 16-byte row chunks: the MFMA layout
    // (a lane holds one column of 4 rows) would write each row in 32-byte
    // pieces of 2-byte stores, which cost 2.5-4.6 us of a 9-12 us launch at
    // M = 576..1024.  Same values as store_plain / store_swiglu.
    // (The tiles reuse the fold operands' LDS, so the launch needs no more
    // than the larger of the two: at the 27B-class shapes that keeps 3
    // workgroups per CU instead of 2.  Every wave has read its last fold
    // operand before any wave passes this barrier.)
    constexpr int TR = 16 * WM, TC = EPI == 0 ? 16 * WN : 8 * WN, CPR = TC / 8, NCH = TR * CPR;
    __syncthreads();
    uint16_t* yt = reinterpret_cast<uint16_t*>(lds_f) + wave * TR * TC;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rl = 16 * i + 4 * lgrp + r;
        if constexpr (EPI == 0) {
#pragma unroll
          for (int j = 0; j < WN; ++j) yt[rl * TC + 16 * j + lrow] = ifrd::f2h(asr[i][r] * acc[i][j][r]);
        } else {
#pragma unroll
          for (int j = 0; j < WN; j += 2) {
            const float g = ifrd::fp16r(asr[i][r] * acc[i][j][r]);
            const float u = ifrd::fp16r(asr[i][r] * acc[i][j + 1][r]);
            yt[rl * TC + 8 * j + lrow] = ifrd::f2h(silu_f(g) * u);
          }
        }
      }
    ifrd::wave_sync();
    const int col0 = EPI == 0 ? 16 * tile0 : 8 * tile0;
#pragma unroll
    for (int q = 0; q < (NCH + 63) / 64; ++q) {
      const int ch = lane + 64 * q;
      if (NCH % 64 != 0 && ch >= NCH) break;
      const int rr = ch / CPR, cc = (ch % CPR) * 8, row = row0 + rr;
      const bool colv = EPI == 0 ? tile0 + cc / 16 < ntiles : tile0 + 2 * (cc / 16) + 1 < ntiles;
      const uint4 v = *reinterpret_cast<const uint4*>(yt + rr * TC + cc);
      if (row < p.M && colv) *reinterpret_cast<uint4*>(p.out + (size_t)row * p.ldo + col0 + cc) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 16 * i + 4 * lgrp + r;
      if (row >= p.M) continue;
      if constexpr (EPI == 0) {
#pragma unroll
        for (int j = 0; j < WN; ++j)
          if (tile0 + j < ntiles) store_plain(p, row, 16 * (tile0 + j) + lrow, asr[i][r], acc[i][j][r]);
      } else {
#pragma unroll
        for (int j = 0; j < WN; j += 2)
          if (tile0 + j + 1 < ntiles)
            store_swiglu(p, row, 16 * ((tile0 + j) >> 1) + lrow, asr[i][r], acc[i][j][r],
                         acc[i][j + 1][r]);
      }
    }
}

// ---- larger M: a workgroup computes a BM x BN block, its 4 waves arranged
// MW x (4/MW); each wave owns WM x WN 16x16 tiles and folds its own
// accumulators group by group while the next R groups are in flight.  The
// loads are unconditional (R divides ng; the last R groups are peeled), so the
// wait before each group only covers that group's operands.
// MODE 0: the general fold; 1: the general fold, T dumped; 2: the codebook fold.
template <int BITS, int WM, int WN, int MW, int R, int EPI, int MODE>
__global__ __launch_bounds__(256) void qgemm_rows(KParams p) {
  constexpr bool DUMP = MODE == 1, FF = MODE == 2;
  constexpr int NW = 4 / MW;
  constexpr int BM = 16 * WM * MW, BN = 16 * WN * NW;
  // (declared as 16-byte vectors so the dynamic LDS is 16-byte aligned and
  // the compiler may use 128-bit LDS accesses)
  extern __shared__ v4f lds_f4[];
  float* const lds_f = reinterpret_cast<float*>(lds_f4);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.N >> 4, ng = p.ng;
  int bx = blockIdx.x, by = blockIdx.y;
  if (p.swz != 0) {
    const bool cols = p.swz > 0;
    const int own = cols ? p.nbx : p.nby, other = cols ? p.nby : p.nbx;
    const int x = blockIdx.x & 7, local = blockIdx.x >> 3, per = (own + 7) >> 3;
    const int G = min(cols ? p.swz : -p.swz, per);
    const int gi = local / (G * other), r = local - gi * G * other;
    const int Gg = min(G, per - gi * G);
    const int o = r / Gg, w = x + 8 * (gi * G + (r - o * Gg));
    bx = cols ? w : o;
    by = cols ? o : w;
    if (bx >= p.nbx || by >= p.nby) return;  // padding (before any barrier)
  }
  const int bm0 = by * BM, bt0 = bx * (BN / 16);
  const int wm = wave % MW, wn = wave / MW;
  const int row0 = bm0 + 16 * WM * wm, tile0 = bt0 + WN * wn;
  float* S_l = lds_f;
  uint32_t* Z_l = reinterpret_cast<uint32_t*>(lds_f + ng * BM);

  uint32_t aoff[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) aoff[i] = (uint32_t)((min(row0 + 16 * i, p.M - 1) >> 4) * p.nsteps * 1024 + 16 * lane);
  int tl[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) tl[j] = min(tile0 + j, ntiles - 1);

  using Ops = GroupOps<BITS, WM, WN>;
  Ops ring[R];
#pragma unroll
  for (int d = 0; d < R; ++d) load_ops<BITS, WM, WN>(p, aoff, tl, lane, d, ring[d]);
  stage_fold_operands<BM, BN, 12, BITS, FF>(p, bm0, bt0, S_l, Z_l);
  float asr[WM][4];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) asr[i][r] = p.as[min(row0 + 16 * i + 4 * lgrp + r, p.M - 1)] * p.post;
  __syncthreads();  // the operands' barrier (the 16-byte store path has one more)

  v4i T[WM][WN];
  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  auto fold = [&](int g) {
    v4f S[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i)
      S[i] = *reinterpret_cast<const v4f*>(&S_l[g * BM + 16 * WM * wm + 16 * i + 4 * lgrp]);
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const uint32_t zw = Z_l[g * BN + 16 * (WN * wn + j) + lrow];
      if constexpr (FF) {  // S holds Y, zw the scale / 2
        const float h = __uint_as_float(zw);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][r] = fmaf(h, __int_as_float(T[i][j][r]) - S[i][r], acc[i][j][r]);
        continue;
      }
      const float sc = ifrd::h2f((uint16_t)(zw & 0xFFFFu));
      const float ze = ifrd::h2f((uint16_t)(zw >> 16));
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int32_t Tv = true_t<BITS>(T[i][j][r], S[i][r]);
          const float d = fmaf(-ze, S[i][r], (float)Tv);
          acc[i][j][r] = fmaf(sc, d, acc[i][j][r]);
          if (DUMP && row0 + 16 * i + 4 * lgrp + r < p.M && tile0 + j < ntiles)
            p.tdump[((size_t)(row0 + 16 * i + 4 * lgrp + r) * p.N + 16 * tl[j] + lrow) * ng + g] = Tv;
        }
    }
  };
  int g = 0;
  for (; g + R < ng; g += R) {
#pragma unroll
    for (int d = 0; d < R; ++d) {
      mma_group<BITS, WM, WN, FF>(ring[d], T);
      load_ops<BITS, WM, WN>(p, aoff, tl, lane, g + d + R, ring[d]);
      fold(g + d);
    }
  }
#pragma unroll
  for (int d = 0; d < R; ++d) {
    mma_group<BITS, WM, WN, FF>(ring[d], T);
    fold(g + d);
  }

  if constexpr (EPI == 2) {
    qk_epilogue<BM, BN, WM, WN, MW>(p, lds_f, acc, asr, bm0, bt0, wave, lane);
    return;
  }
  if (!DUMP && p.vst) {
    // The wave's output tile (16 WM rows x TC columns of fp16) is staged in
    // its own LDS slice and stored as 16-byte row chunks: the MFMA layout
    // (a lane holds one column of 4 rows) would write each row in 32-byte
    // pieces of 2-byte stores, which cost 2.5-4.6 us of a 9-12 us launch at
    // M = 576..1024.  Same values as store_plain / store_swiglu.
    // (The tiles reuse the fold operands' LDS, so the launch needs no more
    // than the larger of the two: at the 27B-class shapes that keeps 3
    // workgroups per CU instead of 2.  Every wave has read its last fold
    // operand before any wave passes this barrier.)
    constexpr int TR = 16 * WM, TC = EPI == 0 ? 16 * WN : 8 * WN, CPR = TC / 8, NCH = TR * CPR;
    __syncthreads();
    uint16_t* yt = reinterpret_cast<uint16_t*>(lds_f) + wave * TR * TC;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rl = 16 * i + 4 * lgrp + r;
        if constexpr (EPI == 0) {
#pragma unroll
          for (int j = 0; j < WN; ++j) yt[rl * TC + 16 * j + lrow] = ifrd::f2h(asr[i][r] * acc[i][j][r]);
        } else {
#pragma unroll
          for (int j = 0; j < WN; j += 2) {
            const float g = ifrd::fp16r(asr[i][r] * acc[i][j][r]);
            const float u = ifrd::fp16r(asr[i][r] * acc[i][j + 1][r]);
            yt[rl * TC + 8 * j + lrow] = ifrd::f2h(silu_f(g) * u);
          }
        }
      }
    ifrd::wave_sync();
    const int col0 = EPI == 0 ? 16 * tile0 : 8 * tile0;
#pragma unroll
    for (int q = 0; q < (NCH + 63) / 64; ++q) {
      const int ch = lane + 64 * q;
      if (NCH % 64 != 0 && ch >= NCH) break;
      const int rr = ch / CPR, cc = (ch % CPR) * 8, row = row0 + rr;
      const bool colv = EPI == 0 ? tile0 + cc / 16 < ntiles : tile0 + 2 * (cc / 16) + 1 < ntiles;
      const uint4 v = *reinterpret_cast<const uint4*>(yt + rr * TC + cc);
      if (row < p.M && colv) *reinterpret_cast<uint4*>(p.out + (size_t)row * p.ldo + col0 + cc) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 16 * i + 4 * lgrp + r;
      if (row >= p.M) continue;
      if constexpr (EPI == 0) {
#pragma unroll
        for (int j = 0; j < WN; ++j)
          if (tile0 + j < ntiles) store_plain(p, row, 16 * (tile0 + j) + lrow, asr[i][r], acc[i][j][r]);
      } else {
#pragma unroll
        for (int j = 0; j < WN; j += 2)
          if (tile0 + j + 1 < ntiles)
            store_swiglu(p, row, 16 * ((tile0 + j) >> 1) + lrow, asr[i][r], acc[i][j][r],
                         acc[i][j + 1][r]);
      }
    }
}

// ---- mid M (the mixed-iteration shapes, K up to a few thousand): every
// memory access of the K loop is issued at kernel entry, so a wave waits for
// memory once instead of once per R groups.  The workgroup's A rows for the
// whole K (BM x K bytes) go to LDS by the LDS DMA (global_load_lds_dwordx4:
// one contiguous 1 KB A tile per wave instruction, no VGPRs; the waves of a
// row block share it instead of each loading the same fragments), each
// wave's B codes for all NG = ng groups go to registers, and the fold
// operands are staged as in qgemm_rows.  After one wait and one barrier the
// K loop reads A from LDS, runs the MFMAs and folds group by group in
// ascending order, so the bits are those of every other launch shape.  The
// scale | zero pairs of the wave's own columns are loaded into registers
// with the codes (NG x WN of them) instead of LDS, which keeps the 16-row
// block of the 24-group down projection at 3 workgroups per CU.
template <int BITS, int WM, int WN, int MW, int NG, int EPI, int MODE>
__global__ __launch_bounds__(256) void qgemm_full(KParams p) {
  constexpr bool DUMP = MODE == 1, FF = MODE == 2;
  constexpr int NW = 4 / MW;
  constexpr int BM = 16 * WM * MW, BN = 16 * WN * NW, NS = 2 * NG;
  constexpr int NCHUNK = (BM / 16) * NS;  // 1 KB A tiles of the block
  static_assert(NCHUNK % 4 == 0, "the waves share the A copies evenly");
  extern __shared__ v4f lds_f4[];
  float* const lds_f = reinterpret_cast<float*>(lds_f4);
  int8_t* const A_l = reinterpret_cast<int8_t*>(lds_f4);  // [BM / 16][NS][1 KB]
  float* const S_l = reinterpret_cast<float*>(A_l + NCHUNK * 1024);  // [NG][BM]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.N >> 4;
  const int bm0 = blockIdx.y * BM, bt0 = blockIdx.x * (BN / 16);
  const int wm = wave % MW, wn = wave / MW;
  const int row0 = bm0 + 16 * WM * wm, tile0 = bt0 + WN * wn;

  // A: chunk c = rt * NS + s is row tile rt's K step s (row tiles past the
  // last one read the last, whose outputs are never stored)
  const int last_rt = (p.M - 1) >> 4;
#pragma unroll
  for (int q = 0; q < NCHUNK / 4; ++q) {
    const int c = wave + 4 * q, rt = c / NS, s = c - rt * NS;
    const int8_t* src = p.a + ((size_t)min((bm0 >> 4) + rt, last_rt) * NS + s) * 1024 + 16 * lane;
    __builtin_amdgcn_global_load_lds(src, A_l + c * 1024, 16, 0, 0);
  }
  int tl[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) tl[j] = min(tile0 + j, ntiles - 1);
  uint32_t Bw[NG][2][WN][BITS / 2];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < WN; ++j)
        load_raw<BITS>(p.codes + ((size_t)tl[j] * NS + 2 * g + h) * 64 * (BITS / 2), lane, Bw[g][h][j]);
  uint32_t zr[NG][WN];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int j = 0; j < WN; ++j) zr[g][j] = p.sz[((size_t)tl[j] * NG + g) * 16 + lrow];
  {
    // S (FF: Y = 1.5 * 2^23 + C * S) of the block's rows, [NG][BM]; rows
    // past M read row M - 1 (their outputs are never stored)
    constexpr float C = (float)((1 << BITS) - 1);
    constexpr int NQ = (NG * BM + 255) / 256;
    float sv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + 256 * q;
      if (t < NG * BM) sv[q] = p.gs[(size_t)min(bm0 + t % BM, p.M - 1) * NG + t / BM];
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + 256 * q;
      if (t < NG * BM) S_l[t] = FF ? kFoldBiasF + C * sv[q] : sv[q];
    }
  }
  float asr[WM][4];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) asr[i][r] = p.as[min(row0 + 16 * i + 4 * lgrp + r, p.M - 1)] * p.post;
  // the LDS copies are counted by vmcnt: every wave's must land before any
  // wave reads A
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  v4i T[WM][WN];
  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    GroupOps<BITS, WM, WN> ops;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < WM; ++i)
        ops.A[h][i] = *reinterpret_cast<const v4i*>(A_l + ((wm * WM + i) * NS + 2 * g + h) * 1024 + 16 * lane);
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int q = 0; q < BITS / 2; ++q) ops.B[h][j][q] = Bw[g][h][j][q];
    }
    mma_group<BITS, WM, WN, FF>(ops, T);
    fold_group<BITS, WM, WN, MW, FF, DUMP>(p, S_l, zr[g], T, acc, g, wm, wn, lane, row0, tile0, tl);
  }
  if constexpr (EPI == 2) {
    qk_epilogue<BM, BN, WM, WN, MW>(p, lds_f, acc, asr, bm0, bt0, wave, lane);
    return;
  }
  store_tiles<WM, WN, EPI, DUMP>(p, lds_f, acc, asr, row0, tile0, wave, lane);
}

// ---- small M (decode, weight-stream bound): the 4 waves split the K groups
// of one WM x WN tile block.  Each wave issues the loads of all its groups
// (at most NGW) at entry, runs the MFMAs, and parks its int32 T in LDS; after
// one barrier all 256 lanes fold every group in ascending order.
template <int BITS, int WM, int WN, int NGW, int EPI, int MODE>
__global__ __launch_bounds__(256) void qgemm_splitk(KParams p) {
  constexpr bool DUMP = MODE == 1, FF = MODE == 2;
  extern __shared__ v4i lds4[];  // 16-byte aligned: T parks as 128-bit stores
  int32_t* const lds = reinterpret_cast<int32_t*>(lds4);
  constexpr int BM = 16 * WM, BN = 16 * WN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int ntiles = p.N >> 4, ng = p.ng;
  const int row0 = blockIdx.y * BM;
  const int tile0 = blockIdx.x * WN;
  const int g0 = (ng * wave) / 4, g1 = (ng * (wave + 1)) / 4;
  uint32_t aoff[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) aoff[i] = (uint32_t)((min(row0 + 16 * i, p.M - 1) >> 4) * p.nsteps * 1024 + 16 * lane);
  int tl[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) tl[j] = min(tile0 + j, ntiles - 1);
  float* S_l = reinterpret_cast<float*>(lds + (size_t)ng * WM * WN * 256);
  uint32_t* Z_l = reinterpret_cast<uint32_t*>(S_l + BM * ng);

  using Ops = GroupOps<BITS, WM, WN>;
  Ops ops[NGW];
  // A wave can own no group (ng < 4); it then loads group 0, whose result it
  // never uses, so every load stays inside the operands.
  const int glast = max(g1 - 1, 0);
#pragma unroll
  for (int d = 0; d < NGW; ++d) load_ops<BITS, WM, WN>(p, aoff, tl, lane, min(g0 + d, glast), ops[d]);
  stage_fold_operands<BM, BN, 6, BITS, FF>(p, row0, tile0, S_l, Z_l);
  constexpr int JS = (EPI == 0) ? 1 : 2;  // swiglu: one thread folds the pair
  constexpr int NOUT = WM * (WN / JS) * 256;
  constexpr int NO = (NOUT + 255) / 256;
  float asv[NO];
#pragma unroll
  for (int k = 0; k < NO; ++k) {
    const int o = threadIdx.x + 256 * k;
    const int r = o & 3, ln = (o >> 2) & 63, i = (o >> 8) / (WN / JS);
    asv[k] = p.as[min(row0 + 16 * i + 4 * (ln >> 4) + r, p.M - 1)] * p.post;
  }
  v4i T[WM][WN];
#pragma unroll
  for (int d = 0; d < NGW; ++d) {
    if (g0 + d < g1) {
      mma_group<BITS, WM, WN, FF>(ops[d], T);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          *reinterpret_cast<v4i*>(&lds[(((size_t)(g0 + d) * WM + i) * WN + j) * 256 + lane * 4]) = T[i][j];
    }
  }
  __syncthreads();
  // Fold all groups in order.  Output o = ((i*(WN/JS) + jj/JS)*64 + lane')*4 + r.
#pragma unroll
  for (int k = 0; k < NO; ++k) {
    const int o = threadIdx.x + 256 * k;
    if (o >= NOUT) break;
    const int r = o & 3, ln = (o >> 2) & 63, ij = o >> 8;
    const int jj = (ij % (WN / JS)) * JS, i = ij / (WN / JS);
    const int rl = 16 * i + 4 * (ln >> 4) + r, row = row0 + rl;
    const int c = ln & 15;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
    for (int g = 0; g < ng; ++g) {
      const float S = S_l[g * BM + rl];
#pragma unroll
      for (int q = 0; q < JS; ++q) {
        const int j = jj + q;
        const int32_t Tr = lds[(((size_t)g * WM + i) * WN + j) * 256 + ln * 4 + r];
        const uint32_t szw = Z_l[g * BN + 16 * j + c];
        if constexpr (FF) {  // S holds Y, szw the scale / 2
          const float d2 = __int_as_float(Tr) - S;
          if (q == 0) a0 = fmaf(__uint_as_float(szw), d2, a0); else a1 = fmaf(__uint_as_float(szw), d2, a1);
          continue;
        }
        const int32_t Tv = true_t<BITS>(Tr, S);
        const float sc = ifrd::h2f((uint16_t)(szw & 0xFFFFu));
        const float ze = ifrd::h2f((uint16_t)(szw >> 16));
        const float d = fmaf(-ze, S, (float)Tv);
        if (q == 0) a0 = fmaf(sc, d, a0); else a1 = fmaf(sc, d, a1);
        if (DUMP && row < p.M && tile0 + j < ntiles)
          p.tdump[((size_t)row * p.N + 16 * tl[j] + c) * ng + g] = Tv;
      }
    }
    if (row >= p.M) continue;
    if constexpr (EPI == 0) {
      if (tile0 + jj < ntiles) store_plain(p, row, 16 * (tile0 + jj) + c, asv[k], a0);
    } else {
      if (tile0 + jj + 1 < ntiles) store_swiglu(p, row, 16 * ((tile0 + jj) >> 1) + c, asv[k], a0, a1);
    }
  }
}

// ---- decode on large weights (M <= 16): the weight stream.  A workgroup of
// NWV waves owns WN column tiles over the whole K; wave w takes the K groups
// [ng w / NWV, ng (w + 1) / NWV) (at most NGW) through a ring of P groups
// of codes: a group's slot is refilled with the group P ahead as soon as
// its MFMAs have read it, so the fold of arrived groups overlaps the stream
// of the rest.  The code loads are the only vector-memory instructions per
// group: the scale | zero pairs of the wave's groups arrive at entry, four
// groups x 16 columns per load, and reach the lanes that fold a group by a
// lane permute; the A rows come from LDS where M <= 4 (the block fetches
// the M rows of the whole K once, ALDS), else per group with the codes.
// Only real rows are fetched and folded: A fragments of rows >= M are zero,
// and a lane's row quad runs min(4, M) fold steps.  Each wave turns the T of
// its groups into d = fma(-zero, S, T) right after the MFMAs and parks d in
// one row per output (groups along the row, pitch p.spitch) and the group's
// scale as fp32 in one row per column; after the last barrier each output
// runs the dependent chain acc = fma(scale, d, acc) along its row, groups
// ascending, four groups per 128-bit LDS read.  Each wave stages S and the
// ALDS rows of its own groups in its own LDS region, so no workgroup barrier
// precedes the ring.
template <int BITS, int WN, int NWV, int NGW, int P, int EPI, bool ALDS, bool DUMP>
__global__ __launch_bounds__(64 * NWV) void qgemm_stream(KParams p) {
  extern __shared__ v4i lds4[];  // 16-byte aligned: the rows are read 128 bits at a time
  float* const D_l = reinterpret_cast<float*>(lds4);  // [M][BN][gp] d
  constexpr int BN = 16 * WN, NT = 64 * NWV;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ntiles = p.N >> 4, ng = p.ng, M = p.M, gp = p.spitch;
  const int tile0 = blockIdx.x * WN;
  const int g0 = (ng * wave) / NWV, g1 = (ng * (wave + 1)) / NWV;
  int tl[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) tl[j] = min(tile0 + j, ntiles - 1);
  float* const C_l = D_l + (size_t)M * BN * gp;  // [BN][gp] fp32 scale
  // each wave's own operands: S of its groups [NGW][16] and, ALDS, its A
  // rows [M][8 NGW chunks of 16 bytes] (the chunks (step, quarter) of its
  // groups, in row-major order)
  float* const S_w = C_l + (size_t)BN * gp + (size_t)wave * 16 * NGW;
  int8_t* const As_w = reinterpret_cast<int8_t*>(C_l + (size_t)BN * gp + (size_t)NWV * 16 * NGW) +
                       (size_t)wave * M * 128 * NGW;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int glast = max(g1 - 1, 0), ngw = g1 - g0;

  // S: item t = (group gi = t / 16, row r = t % 16)
  constexpr int SQ = (16 * NGW + 63) / 64;
  float sv[SQ];
#pragma unroll
  for (int q = 0; q < SQ; ++q) {
    const int t = lane + 64 * q, gi = t >> 4, r = t & 15;
    sv[q] = (r < M && gi < ngw) ? p.gs[(size_t)r * ng + g0 + gi] : 0.f;
  }
  // ALDS: item t = (row r, chunk c = 4 step + quarter of the wave's steps),
  // from p.arow when given (contiguous), else gathered from the A tiles (16
  // useful bytes per 128-byte line a row touches)
  constexpr int CW = 8 * NGW, AQ = ALDS ? (4 * CW + 63) / 64 : 1;
  v4i av[AQ];
  if constexpr (ALDS) {
    const bool rows = p.arow != nullptr;
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int t = lane + 64 * q, r = t / CW, c = t % CW;
      const int st = 2 * g0 + (c >> 2), qu = c & 3;
      const int8_t* src = rows ? p.arow + (size_t)r * p.K + 64 * st + 16 * qu
                               : p.a + 1024 * st + 16 * (16 * qu + r);
      av[q] = (r < M && (c >> 3) < ngw) ? *reinterpret_cast<const v4i*>(src) : (v4i){0, 0, 0, 0};
    }
  }
  // scale | zero pairs: load q of tile j holds groups g0 + 4q .. + 3 (lane
  // group lgrp) x the 16 columns (lane row).  Issued after S and the ALDS
  // rows (L2-resident), so that staging those waits for them alone, not for
  // these first reads of the weights.
  constexpr int ZW = (NGW + 3) / 4;
  uint32_t zq[WN][ZW];
#pragma unroll
  for (int q = 0; q < ZW; ++q)
#pragma unroll
    for (int j = 0; j < WN; ++j)
      zq[j][q] = p.sz[((size_t)tl[j] * ng + min(g0 + 4 * q + lgrp, glast)) * 16 + lrow];
  // the ring: group d of the wave in slot d % P.  Loads are unconditional
  // (past the wave's last group they repeat it) so that the wait before each
  // group covers only that group's operands.
  const bool arow = lrow < M;
  GroupOps<BITS, 1, WN> ring[P];
  auto fetch = [&](int d, GroupOps<BITS, 1, WN>& o) {
    const int g = min(g0 + d, glast);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int st = 2 * g + h;
      if constexpr (!ALDS)
        o.A[h][0] = arow ? *reinterpret_cast<const v4i*>(p.a + 1024 * st + 16 * lane) : (v4i){0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < WN; ++j)
        load_raw<BITS>(p.codes + ((size_t)tl[j] * p.nsteps + st) * 64 * (BITS / 2), lane, o.B[h][j]);
    }
  };
#pragma unroll
  for (int d = 0; d < P && d < NGW; ++d) fetch(d, ring[d]);
#pragma unroll
  for (int q = 0; q < SQ; ++q) {
    const int t = lane + 64 * q;
    if (t < 16 * NGW) S_w[t] = sv[q];
  }
  if constexpr (ALDS) {
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int t = lane + 64 * q, r = t / CW, c = t % CW;
      if (r < M) *reinterpret_cast<v4i*>(As_w + ((size_t)r * CW + c) * 16) = av[q];
    }
  }
  // the wave's own LDS regions: no workgroup barrier before the ring
  ifrd::wave_sync();
  // this lane's real rows: 4 lgrp .. 4 lgrp + rq - 1; the fold steps run to
  // the wave-uniform min(4, M)
  const int rq = M - 4 * lgrp, rmax = min(4, M);
  // The LDS operands of group d + 1 (ALDS rows, S, the permuted scale | zero
  // pairs) are read while group d folds: issued after group d's MFMAs and
  // before its stores, in program order, so they are in registers when
  // group d + 1 starts.
  v4i an[2];
  v4f Sn;
  uint32_t zn[WN];
  auto lds_ops = [&](int d) {
    if constexpr (ALDS) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        an[h] = arow ? *reinterpret_cast<const v4i*>(As_w + ((size_t)lrow * CW + (2 * d + h) * 4 + lgrp) * 16)
                     : (v4i){0, 0, 0, 0};
    }
    Sn = *reinterpret_cast<const v4f*>(&S_w[d * 16 + 4 * lgrp]);
#pragma unroll
    for (int j = 0; j < WN; ++j) zn[j] = (uint32_t)__shfl((int)zq[j][d >> 2], lrow + 16 * (d & 3), 64);
  };
  lds_ops(0);
#pragma unroll
  for (int d = 0; d < NGW; ++d) {
    GroupOps<BITS, 1, WN>& o = ring[d % P];
    const int g = g0 + d;
    if constexpr (ALDS) {
      o.A[0][0] = an[0];
      o.A[1][0] = an[1];
    }
    const v4f S4 = Sn;
    uint32_t zw[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) zw[j] = zn[j];
    v4i T[1][WN];
    mma_group<BITS, 1, WN>(o, T);
    if (d + P < NGW) fetch(d + P, o);
    if (d + 1 < NGW) lds_ops(d + 1);
    if (g < g1) {
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if (lgrp == 0) C_l[(size_t)(16 * j + lrow) * gp + g] = ifrd::h2f((uint16_t)(zw[j] & 0xFFFFu));
        const float ze = ifrd::h2f((uint16_t)(zw[j] >> 16));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r < rmax && r < rq) {
            const int32_t Tv = true_t<BITS>(T[0][j][r], S4[r]);
            D_l[((size_t)(4 * lgrp + r) * BN + 16 * j + lrow) * gp + g] = fmaf(-ze, S4[r], (float)Tv);
            if (DUMP && tile0 + j < ntiles)
              p.tdump[((size_t)(4 * lgrp + r) * p.N + 16 * tl[j] + lrow) * ng + g] = Tv;
          }
        }
      }
    }
  }
  __syncthreads();
  // outputs o = (pair jp, row, column c) over 256-slot pair blocks; slots
  // of rows >= M idle
  constexpr int JS = (EPI == 0) ? 1 : 2;  // swiglu: one thread folds the pair
  for (int o = threadIdx.x; o < 256 * (WN / JS); o += NT) {
    const int c = o & 15, row = (o >> 4) & 15, jj = (o >> 8) * JS;
    if (row >= M) continue;
    const float* d0 = D_l + ((size_t)row * BN + 16 * jj + c) * gp;
    const float* s0 = C_l + (size_t)(16 * jj + c) * gp;
    const float* d1 = d0 + (JS == 2 ? 16 * gp : 0);
    const float* s1 = s0 + (JS == 2 ? 16 * gp : 0);
    float a0 = 0.f, a1 = 0.f;
    int g = 0;
#pragma unroll 4
    for (; g + 4 <= ng; g += 4) {
      const v4f dv = *reinterpret_cast<const v4f*>(d0 + g), sc = *reinterpret_cast<const v4f*>(s0 + g);
      a0 = fmaf(sc.x, dv.x, a0);
      a0 = fmaf(sc.y, dv.y, a0);
      a0 = fmaf(sc.z, dv.z, a0);
      a0 = fmaf(sc.w, dv.w, a0);
      if constexpr (JS == 2) {
        const v4f dw = *reinterpret_cast<const v4f*>(d1 + g), sw = *reinterpret_cast<const v4f*>(s1 + g);
        a1 = fmaf(sw.x, dw.x, a1);
        a1 = fmaf(sw.y, dw.y, a1);
        a1 = fmaf(sw.z, dw.z, a1);
        a1 = fmaf(sw.w, dw.w, a1);
      }
    }
    for (; g < ng; ++g) {
      a0 = fmaf(s0[g], d0[g], a0);
      if constexpr (JS == 2) a1 = fmaf(s1[g], d1[g], a1);
    }
    const float as = p.as[row] * p.post;
    if constexpr (EPI == 0) {
      if (tile0 + jj < ntiles) store_plain(p, row, 16 * (tile0 + jj) + c, as, a0);
    } else {
      if (tile0 + jj + 1 < ntiles) store_swiglu(p, row, 16 * ((tile0 + jj) >> 1) + c, as, a0, a1);
    }
  }
}

template <typename F>
hipError_t set_lds_limit(F* f) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize,
                             160 * 1024);
}

template <int BITS, int WM, int WN, int MW, int R, int EPI>
hipError_t launch_rows(const KParams& p, hipStream_t st) {
  constexpr int NW = 4 / MW;
  constexpr int BM = 16 * WM * MW, BN = 16 * WN * NW;
  if (p.ng % R != 0) return hipErrorInvalidValue;
  size_t lds = (size_t)p.ng * (BM + BN) * sizeof(float);
  // the output tiles of the 4 waves (16-byte stores), in the same space
  if constexpr (EPI != 2) lds = std::max(lds, (size_t)4 * 16 * WM * (EPI == 0 ? 16 * WN : 8 * WN) * sizeof(uint16_t));
  if constexpr (EPI == 2) {
    // the staged y tile (padded rows) and the RMS partial sums
    if (BM != 32 || BN != 128 || p.qa.rotary != 128 || p.kv.hd != 128) return hipErrorInvalidValue;
    lds = std::max(lds, (size_t)(BM * (BN + 4) + BM * 8) * sizeof(float));
  }
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  constexpr bool kFF = BITS != 8;  // the codebook fold needs 2c in int8
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = set_lds_limit(qgemm_rows<BITS, WM, WN, MW, R, EPI, 0>);
    if constexpr (EPI == 0)
      if (e == hipSuccess) e = set_lds_limit(qgemm_rows<BITS, WM, WN, MW, R, EPI, 1>);
    if constexpr (kFF)
      if (e == hipSuccess) e = set_lds_limit(qgemm_rows<BITS, WM, WN, MW, R, EPI, 2>);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int ntiles = p.N / 16;
  KParams q = p;
  q.vst = EPI != 2 && !p.tdump && reinterpret_cast<uintptr_t>(p.out) % 16 == 0 && p.ldo % 8 == 0;
  q.nbx = (ntiles + BN / 16 - 1) / (BN / 16);
  q.nby = (p.M + BM - 1) / BM;
  // XCD-grouped order by weight columns when an XCD's share of the weights
  // would not stay in its 4 MB L2, in groups that fill about 2 MB
  // (bench.py --cfg5: gate/up 56.7 -> 54 ms; no gain below that size).
  // Grouping by activation rows instead (swz < 0) made the 27B down
  // projection, whose A is larger than its weights, slower (32.6 -> 38.7
  // ms), so the host does not choose it.
  const size_t colblock_bytes = (size_t)BN * p.K * BITS / 8 + (size_t)BN * p.ng * 4;
  const size_t mb2 = (size_t)2 << 20, mb3 = (size_t)3 << 20;
  q.swz = (q.nbx >= 8 && q.nby >= 2 && (size_t)((q.nbx + 7) / 8) * colblock_bytes > mb3)
              ? (int)std::max<size_t>(1, mb2 / colblock_bytes) : 0;
  const dim3 grid = q.swz > 0 ? dim3((q.nbx + 7) / 8 * 8 * q.nby)
                    : q.swz < 0 ? dim3((q.nby + 7) / 8 * 8 * q.nbx) : dim3(q.nbx, q.nby);
  if constexpr (EPI == 0)
    if (p.tdump) {
      hipLaunchKernelGGL((qgemm_rows<BITS, WM, WN, MW, R, EPI, 1>), grid, dim3(256), lds, st, q);
      return hipGetLastError();
    }
  if constexpr (kFF)
    if (p.ff) {
      hipLaunchKernelGGL((qgemm_rows<BITS, WM, WN, MW, R, EPI, 2>), grid, dim3(256), lds, st, q);
      return hipGetLastError();
    }
  hipLaunchKernelGGL((qgemm_rows<BITS, WM, WN, MW, R, EPI, 0>), grid, dim3(256), lds, st, q);
  return hipGetLastError();
}

template <int BITS, int WM, int WN, int NGW, int EPI>
hipError_t launch_splitk(const KParams& p, hipStream_t st) {
  const int ntiles = p.N / 16;
  const dim3 grid((ntiles + WN - 1) / WN, (p.M + 16 * WM - 1) / (16 * WM));
  const size_t lds = ((size_t)p.ng * WM * WN * 256 + (size_t)16 * (WM + WN) * p.ng) * sizeof(int32_t);
  if ((p.ng + 3) / 4 > NGW || lds > 160 * 1024) return hipErrorInvalidValue;
  constexpr bool kFF = BITS != 8;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = set_lds_limit(qgemm_splitk<BITS, WM, WN, NGW, EPI, 0>);
    if constexpr (EPI == 0)
      if (e == hipSuccess) e = set_lds_limit(qgemm_splitk<BITS, WM, WN, NGW, EPI, 1>);
    if constexpr (kFF)
      if (e == hipSuccess) e = set_lds_limit(qgemm_splitk<BITS, WM, WN, NGW, EPI, 2>);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  if constexpr (EPI == 0)
    if (p.tdump) {
      hipLaunchKernelGGL((qgemm_splitk<BITS, WM, WN, NGW, EPI, 1>), grid, dim3(256), lds, st, p);
      return hipGetLastError();
    }
  if constexpr (kFF)
    if (p.ff) {
      hipLaunchKernelGGL((qgemm_splitk<BITS, WM, WN, NGW, EPI, 2>), grid, dim3(256), lds, st, p);
      return hipGetLastError();
    }
  hipLaunchKernelGGL((qgemm_splitk<BITS, WM, WN, NGW, EPI, 0>), grid, dim3(256), lds, st, p);
  return hipGetLastError();
}

template <int BITS, int WM, int WN, int EPI>
hipError_t launch_splitk_ng(const KParams& p, hipStream_t st) {
  const int per = (p.ng + 3) / 4;
  if (per <= 2) return launch_splitk<BITS, WM, WN, 2, EPI>(p, st);
  if (per <= 4) return launch_splitk<BITS, WM, WN, 4, EPI>(p, st);
  if (WM <= 2 && per <= 6) return launch_splitk<BITS, WM, WN, 6, EPI>(p, st);
  return hipErrorInvalidValue;
}

template <int BITS, int WN, int NWV, int NGW, int EPI>
hipError_t launch_stream(const KParams& p, hipStream_t st) {
  // P groups in the ring: the operand registers per group (WN * BITS for the
  // codes, and 8 for A unless ALDS) times P, beside the staging registers
  // (S, the scale | zero pairs, the ALDS rows), T, S and the addresses
  // (24 + 4 WN, and 4 WN more for the SwiGLU tail, as the compiler's counts
  // show), fit the VGPRs of a 64 * NWV-thread workgroup.
  constexpr int kLim = NWV >= 16 ? 120 : 232;
  constexpr int kOver = 24 + 4 * WN + (EPI == 1 ? 4 * WN : 0) + WN * ((NGW + 3) / 4) + (NGW + 3) / 4;
  constexpr int kRing = kStreamRing < NGW ? kStreamRing : NGW;
  constexpr int kFitF = (kLim - kOver) / (8 + WN * BITS);
  constexpr int kFitA = (kLim - kOver - 4 * ((NGW + 1) / 2)) / (WN * BITS);
  constexpr int PF = kRing < kFitF ? kRing : kFitF, PA = kRing < kFitA ? kRing : kFitA;
  if (p.M > 16 || (p.ng + NWV - 1) / NWV > NGW) return hipErrorInvalidValue;
  // LDS: d rows [M][BN] and scale rows [BN] (pitch gp), then per wave S
  // [NGW][16] and the ALDS rows [M][NGW x 128 bytes].  gp: a multiple of 4
  // (four groups per 128-bit read) that is 4 mod 8, so the rows of the 16
  // columns of one group start in different banks; the plain multiple of 4
  // where the padded rows do not fit.
  constexpr int BN = 16 * WN;
  auto need = [&](int gp, bool alds) {
    return ((size_t)(p.M + 1) * BN * gp + (size_t)NWV * 16 * NGW) * sizeof(float) +
           (alds ? (size_t)NWV * p.M * 128 * NGW : 0);
  };
  bool alds = PA >= 1 && p.M <= 4;
  if (alds && need((p.ng + 3) & ~3, true) > 160 * 1024) alds = false;
  if (!alds && PF < 1) return hipErrorInvalidValue;
  int gp = ((p.ng + 3) & ~7) + 4;
  if (need(gp, alds) > 160 * 1024) gp = (p.ng + 3) & ~3;
  const size_t lds = need(gp, alds);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipSuccess;
    if constexpr (PF >= 1) {
      e = set_lds_limit(qgemm_stream<BITS, WN, NWV, NGW, PF, EPI, false, false>);
      if constexpr (EPI == 0)
        if (e == hipSuccess) e = set_lds_limit(qgemm_stream<BITS, WN, NWV, NGW, PF, EPI, false, true>);
    }
    if constexpr (PA >= 1) {
      if (e == hipSuccess) e = set_lds_limit(qgemm_stream<BITS, WN, NWV, NGW, PA, EPI, true, false>);
      if constexpr (EPI == 0)
        if (e == hipSuccess) e = set_lds_limit(qgemm_stream<BITS, WN, NWV, NGW, PA, EPI, true, true>);
    }
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  KParams q = p;
  q.spitch = gp;
  const dim3 grid((p.N / 16 + WN - 1) / WN), block(64 * NWV);
  const bool dump = EPI == 0 && p.tdump;
  if (alds) {
    if constexpr (PA >= 1) {
      if (dump) {
        if constexpr (EPI == 0) hipLaunchKernelGGL((qgemm_stream<BITS, WN, NWV, NGW, PA, EPI, true, true>), grid, block, lds, st, q);
      } else {
        hipLaunchKernelGGL((qgemm_stream<BITS, WN, NWV, NGW, PA, EPI, true, false>), grid, block, lds, st, q);
      }
    }
  } else {
    if constexpr (PF >= 1) {
      if (dump) {
        if constexpr (EPI == 0) hipLaunchKernelGGL((qgemm_stream<BITS, WN, NWV, NGW, PF, EPI, false, true>), grid, block, lds, st, q);
      } else {
        hipLaunchKernelGGL((qgemm_stream<BITS, WN, NWV, NGW, PF, EPI, false, false>), grid, block, lds, st, q);
      }
    }
  }
  return hipGetLastError();
}

// NGW: the smallest instantiated depth that holds ceil(ng / NWV) groups
// (17: the 136-group projection over 8 waves).
template <int BITS, int WN, int NWV, int EPI>
hipError_t launch_stream_ng(const KParams& p, hipStream_t st) {
  const int per = (p.ng + NWV - 1) / NWV;
  if (per <= 1) return launch_stream<BITS, WN, NWV, 1, EPI>(p, st);
  if (per <= 2) return launch_stream<BITS, WN, NWV, 2, EPI>(p, st);
  if (per <= 3) return launch_stream<BITS, WN, NWV, 3, EPI>(p, st);
  if (per <= 5) return launch_stream<BITS, WN, NWV, 5, EPI>(p, st);
  if (per <= 9) return launch_stream<BITS, WN, NWV, 9, EPI>(p, st);
  if (per <= 17) return launch_stream<BITS, WN, NWV, 17, EPI>(p, st);
  return hipErrorInvalidValue;
}

// qgemm_full: NG = ng is a template constant (the 0.8B-class depths 8, 16
// and 24 groups), and every wave's B codes for the whole K must fit 64 VGPRs
// (more spill, and make the compiler's AGPR-copy rewrite fail).  LDS: the A
// rows of the whole K and S, 49.5 KB for the 16-row block at 24 groups (3
// workgroups per CU: the 576 blocks of a 576-row down projection in one
// round).
template <int BITS, int WM, int WN, int MW, int NG, int EPI>
hipError_t launch_full_ng(const KParams& p, hipStream_t st) {
  constexpr int NW = 4 / MW;
  constexpr int BM = 16 * WM * MW, BN = 16 * WN * NW;
  if constexpr (NG * 2 * WN * (BITS / 2) > 64) {
    return hipErrorInvalidValue;
  } else {
    size_t lds = (size_t)BM * NG * 128 + (size_t)NG * BM * sizeof(float);
    if constexpr (EPI == 2) {
      if (BM != 32 || BN != 128 || p.qa.rotary != 128 || p.kv.hd != 128) return hipErrorInvalidValue;
      lds = std::max(lds, (size_t)(BM * (BN + 4) + BM * 8) * sizeof(float));
    } else {
      lds = std::max(lds, (size_t)4 * 16 * WM * (EPI == 0 ? 16 * WN : 8 * WN) * sizeof(uint16_t));
    }
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    constexpr bool kFF = BITS != 8;
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = set_lds_limit(qgemm_full<BITS, WM, WN, MW, NG, EPI, 0>);
      if constexpr (EPI == 0)
        if (e == hipSuccess) e = set_lds_limit(qgemm_full<BITS, WM, WN, MW, NG, EPI, 1>);
      if constexpr (kFF)
        if (e == hipSuccess) e = set_lds_limit(qgemm_full<BITS, WM, WN, MW, NG, EPI, 2>);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
    KParams q = p;
    q.vst = EPI != 2 && !p.tdump && reinterpret_cast<uintptr_t>(p.out) % 16 == 0 && p.ldo % 8 == 0;
    const dim3 grid((p.N / 16 + BN / 16 - 1) / (BN / 16), (p.M + BM - 1) / BM);
    if constexpr (EPI == 0)
      if (p.tdump) {
        hipLaunchKernelGGL((qgemm_full<BITS, WM, WN, MW, NG, EPI, 1>), grid, dim3(256), lds, st, q);
        return hipGetLastError();
      }
    if constexpr (kFF)
      if (p.ff) {
        hipLaunchKernelGGL((qgemm_full<BITS, WM, WN, MW, NG, EPI, 2>), grid, dim3(256), lds, st, q);
        return hipGetLastError();
      }
    hipLaunchKernelGGL((qgemm_full<BITS, WM, WN, MW, NG, EPI, 0>), grid, dim3(256), lds, st, q);
    return hipGetLastError();
  }
}

template <int BITS, int WM, int WN, int MW, int EPI>
hipError_t launch_full(const KParams& p, hipStream_t st) {
  if constexpr (BITS == 8) {
    return hipErrorInvalidValue;  // the codes of the whole K do not fit registers
  } else {
    switch (p.ng) {
      case 8: return launch_full_ng<BITS, WM, WN, MW, 8, EPI>(p, st);
      case 16: return launch_full_ng<BITS, WM, WN, MW, 16, EPI>(p, st);
      case 24: return launch_full_ng<BITS, WM, WN, MW, 24, EPI>(p, st);
      default: return hipErrorInvalidValue;
    }
  }
}

// R (K groups in flight per wave) is the largest power of two <= RMAX that
// divides ng.
template <int BITS, int WM, int WN, int MW, int RMAX, int EPI>
hipError_t launch_rows_r(const KParams& p, hipStream_t st) {
  if (RMAX >= 8 && p.ng % 8 == 0) return launch_rows<BITS, WM, WN, MW, (RMAX >= 8 ? 8 : 1), EPI>(p, st);
  if (RMAX >= 4 && p.ng % 4 == 0) return launch_rows<BITS, WM, WN, MW, (RMAX >= 4 ? 4 : 1), EPI>(p, st);
  if (p.ng % 2 == 0) return launch_rows<BITS, WM, WN, MW, 2, EPI>(p, st);
  return launch_rows<BITS, WM, WN, MW, 1, EPI>(p, st);
}

// Launch-shape table.  Every variant computes identical bits; the choice is
// a pure performance decision (variant < 0: the default heuristic).
template <int BITS, int EPI>
hipError_t launch_bits(const KParams& p, int variant, hipStream_t st);

// The QKV projection with the q/k epilogue: the default shape when it is a
// 32 x 128 row block (one head per workgroup), else declined (the caller
// runs the GEMM and the separate q/k pass).
template <int BITS>
hipError_t launch_bits_qk(const KParams& p, int variant, hipStream_t st) {
  if (variant < 0) {
    const int ng = p.ng;
    // the plain-GEMM heuristic of launch_bits for these shapes
    variant = (ng <= 24 && p.M <= 128) ? 0 : 5;
    if (p.K >= 4096 && p.M > 256 && (ng >= 96 || p.M >= 1024 || p.N >= 6144)) variant = -1;
    if (p.K >= 4096 && p.M <= 16) variant = -1;
    // (the whole-K 32 x 128 block, variant 17, holds the epilogue at 234
    // VGPRs against 126 here: slower in the serve load, 12.7 -> 13.4 us)
  }
  switch (variant) {
    case 4: return launch_rows_r<BITS, 2, 2, 1, 4, 2>(p, st);
    case 5: return launch_rows_r<BITS, 2, 2, 1, 2, 2>(p, st);
    case 12: return launch_rows_r<BITS, 2, 2, 1, 8, 2>(p, st);
    case 17: return launch_full<BITS, 2, 2, 1, 2>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <int BITS, int EPI>
hipError_t launch_bits(const KParams& p, int variant, hipStream_t st) {
  constexpr int WNs = EPI == 0 ? 1 : 2;
  if (variant < 0) {
    // Measured on MI355X, cache-cold weights (bench.py --gemm-variants), the
    // 0.8B shapes at M = 128..1024: split-K wins while the K loop is the
    // latency (narrow N up to M = 576 for 16 groups, 256 for 24; wide N up
    // to M = 128); above that 32 x 128 blocks, deeper for narrow N.
    const bool narrow = EPI == 0 && p.N <= 2048;
    const int splitk_max = narrow ? (p.ng <= 16 ? 576 : 256) : 128;
    if (p.ng <= 24 && p.M <= splitk_max) variant = 0;
    else variant = narrow ? 4 : 5;
    // The 27B-class shapes (K >= 4096; bench.py --gemm-variants-27b, M = 512
    // and 2160): the 136-group down projection keeps its A and B tiles
    // resident best in 64 x 64 blocks, 128 x 64 from M = 1024 (M = 2160:
    // 465 -> 449 us); the others gain from 32 x 256 once M or N is large.
    if (p.K >= 4096 && p.M > 256) {
      if (p.ng >= 96) variant = p.M >= 1024 ? 9 : 3;
      else if (p.M >= 1024 || p.N >= 6144) variant = 6;
    }
    // The mixed-iteration shapes (K of 8, 16 or 24 groups, 128 < M <= 1024;
    // bench.py --gemm-variants --gemm-mall, weights MALL-resident as in the
    // serve load): the whole-K blocks with A in LDS, 16 x 128 up to M = 384
    // and 32 x 128 above for the wide projections, 16 x 64 for O up to
    // M = 768 and 32 x 64 above, 16 x 64 for down up to M = 768 (its blocks
    // then fit one round at 3 per CU; deeper than that, 64 x 64 blocks of
    // qgemm_rows).  A shape the whole-K kernel cannot hold (wider codes)
    // keeps the choice above.
    if ((p.ng == 8 || p.ng == 16 || p.ng == 24) && p.M > 128 && p.M <= 1024) {
      int fv = -1;
      if (p.ng == 24) {
        if (narrow) fv = p.M <= 768 ? 16 : 3;
      } else if (p.ng == 16 && narrow) {
        fv = p.M <= 768 ? 16 : 19;
      } else {
        fv = p.M <= 384 ? 18 : 17;
      }
      if (fv >= 0) {
        const hipError_t e = launch_bits<BITS, EPI>(p, fv, st);
        if (e != hipErrorInvalidValue) return e;
      }
    }
    // Decode rows on those shapes (bench.py --gemm-decode-27b, M = 1, 8, 16):
    // the weight stream; for the plain projections two tiles per workgroup
    // up to M = 4, above it one tile (16 waves for the deep down projection,
    // 8 for the others), and one tile pair of 8 waves for the SwiGLU pair up
    // to M = 8.  A shape a stream variant cannot hold (registers or LDS for
    // wider codes) falls back to the next one, then to the choice above.
    if (p.K >= 4096 && p.M <= 16) {
      hipError_t e = hipErrorInvalidValue;
      if (EPI == 1) {
        if (p.M <= 8) e = launch_bits<BITS, EPI>(p, 14, st);
      } else {
        if (p.M <= 4) e = launch_bits<BITS, EPI>(p, 15, st);
        else if (p.ng < 96) e = launch_bits<BITS, EPI>(p, 14, st);
        if (e == hipErrorInvalidValue) e = launch_bits<BITS, EPI>(p, 13, st);
      }
      if (e != hipErrorInvalidValue) return e;
    }
  }
  switch (variant) {
    case 0: return launch_splitk_ng<BITS, 1, WNs, EPI>(p, st);
    case 1: return launch_splitk_ng<BITS, 2, WNs, EPI>(p, st);
    case 2: return launch_splitk_ng<BITS, 4, WNs, EPI>(p, st);
    case 3: return launch_rows_r<BITS, 2, 2, 2, 4, EPI>(p, st);   // 64 x 64 block
    case 4: return launch_rows_r<BITS, 2, 2, 1, 4, EPI>(p, st);   // 32 x 128 block
    case 5: return launch_rows_r<BITS, 2, 2, 1, 2, EPI>(p, st);   // 32 x 128 block, shallow
    case 6: return launch_rows_r<BITS, 2, 4, 1, 2, EPI>(p, st);   // 32 x 256 block
    case 7: return launch_rows_r<BITS, 4, 2, 1, 2, EPI>(p, st);   // 64 x 128 block
    case 8: return launch_splitk_ng<BITS, 2, 2, EPI>(p, st);      // 32 x 32, split K
    case 9: return launch_rows_r<BITS, 4, 2, 2, 2, EPI>(p, st);   // 128 x 64 block
    case 10: return launch_rows_r<BITS, 1, 2, 1, 8, EPI>(p, st);  // 16 x 128 block, deep
    case 11: return launch_rows_r<BITS, 4, 2, 1, 4, EPI>(p, st);  // 64 x 128 block, deep
    case 12: return launch_rows_r<BITS, 2, 2, 1, 8, EPI>(p, st);  // 32 x 128 block, deep
    case 13: return launch_stream_ng<BITS, WNs, 16, EPI>(p, st);  // decode stream, 16 waves
    case 14: return launch_stream_ng<BITS, WNs, 8, EPI>(p, st);   // decode stream, 8 waves
    case 15: return launch_stream_ng<BITS, 2 * WNs, 16, EPI>(p, st);  // 2 tiles, 16 waves
    // A in LDS and every load issued at entry (K of 8, 16 or 24 groups)
    case 16: return launch_full<BITS, 1, WNs, 1, EPI>(p, st);         // 16 x 64 block
    case 17: return launch_full<BITS, 2, 2, 1, EPI>(p, st);           // 32 x 128 block
    case 18: return launch_full<BITS, 1, 2, 1, EPI>(p, st);           // 16 x 128 block
    case 19: return launch_full<BITS, 2, WNs, 1, EPI>(p, st);         // 32 x 64 block
    case 20: return launch_full<BITS, 1, WNs, 2, EPI>(p, st);         // 32 x 32 block
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

#define IFR_QG_CAT2(a, b) a##b
#define IFR_QG_CAT(a, b) IFR_QG_CAT2(a, b)
hipError_t IFR_QG_CAT(launch_b, IFR_QGEMM_BITS)(const KParams& p, int epi, int variant, hipStream_t st) {
  if (epi == 2) return launch_bits_qk<IFR_QGEMM_BITS>(p, variant, st);
  return epi ? launch_bits<IFR_QGEMM_BITS, 1>(p, variant, st) : launch_bits<IFR_QGEMM_BITS, 0>(p, variant, st);
}

}  // namespace qg
#else

using qg::kG;

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
  return launch_qgemm_variant(w, a, -1, st);
}

hipError_t launch_qgemm_qkrope(const DLin& w, const QGemmArgs& a, const QKArgs& qa, const KVLayout& kv, int variant,
                               hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (w.pair || w.K % kG != 0 || w.N % 128 != 0 || !w.codes || !a.a || !a.as || !a.gs || qa.M != a.M ||
      w.N != ((qa.gated ? 2 : 1) * qa.nq + 2 * kv.nkv) * kv.hd || !qa.qout || (qa.gated && !qa.gout) ||
      !kv.kpool || !kv.vpool || !kv.block_table ||
      (kv.kv_int8 && (!kv.kscale || !kv.vscale)))
    return hipErrorInvalidValue;
  qg::KParams p{a.a, a.as, a.gs, w.codes, w.sz, nullptr, nullptr, a.M, w.N, w.K, w.ng, w.nsteps, w.N,
                w.post, 0, 0, 0, w.ff, 0, 0, qa, kv};
  switch (w.bits) {
    case 2: return qg::launch_b2(p, 2, variant, st);
    case 4: return qg::launch_b4(p, 2, variant, st);
    case 8: return qg::launch_b8(p, 2, variant, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qgemm_variant(const DLin& w, const QGemmArgs& a, int variant, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (w.K % kG != 0 || w.N % 16 != 0 || !w.codes || !a.a || !a.as || !a.gs || !a.out)
    return hipErrorInvalidValue;
  if (w.pair && (w.N % 32 != 0 || a.tdump)) return hipErrorInvalidValue;
  qg::KParams p{a.a, a.as, a.gs, w.codes, w.sz, a.out, a.tdump, a.M, w.N, w.K, w.ng, w.nsteps, a.ldo,
                w.post, 0, 0, 0, w.ff, 0, 0, {}, {}, a.arow};
  const int epi = w.pair ? 1 : 0;
  switch (w.bits) {
    case 2: return qg::launch_b2(p, epi, variant, st);
    case 4: return qg::launch_b4(p, epi, variant, st);
    case 8: return qg::launch_b8(p, epi, variant, st);
    default: return hipErrorInvalidValue;
  }
}

#endif
}  // namespace ifrk
