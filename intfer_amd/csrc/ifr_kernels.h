// Host-side launchers of the gfx950 kernels (one .hip file per family).
// Every launcher checks the shapes its kernel assumes before launching and
// returns a hipError_t (hipErrorInvalidValue for a shape it cannot run).
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace ifrk {

// ---- quantized linear in the device MFMA layout ---------------------------
// codes: fragment-major.  For column tile t (16 columns), 64-wide K step s and
// lane l (column 16t + l%16, K range [64s + 16(l/16), +16)), the lane's
// bits/2 dwords sit at ((t * nsteps + s) * 64 + l) * (bits/2).  Inside them
// code j (j = 0..15) of the lane's 16 K values is stored so that a shift and
// a mask yield the int8 operand dword d = j/4 with byte j%4 (see qgemm.hip).
// sz: (scale, zero) fp16 pairs, [ntiles][ngroups][16].
// Int8 GEMM activations are stored as "A tiles": 16 rows x 64 columns per
// 1 KB tile, tiles ordered (row block, column block); inside a tile the 16
// bytes that MFMA lane l = 16 * ((k % 64) / 16) + m % 16 consumes are
// contiguous.  A wave reads one 16 x 64 operand with one coalesced 1 KB load.
// A buffer for M rows holds ceil(M / 16) * 16 rows.
__host__ __device__ inline size_t atile_off(int m, int k, int K) {
  return ((size_t)((m >> 4) * (K >> 6) + (k >> 6)) << 10) + (size_t)((((k & 63) >> 4) << 4) + (m & 15)) * 16 +
         (k & 15);
}
inline size_t atile_bytes(int M, int K) { return (size_t)((M + 15) / 16) * 16 * K; }

struct DLin {
  int N = 0;       // device columns (2 * F for an interleaved gate/up pair)
  int K = 0;
  int bits = 0;
  int ng = 0;      // K / 128
  int nsteps = 0;  // K / 64
  int pair = 0;    // 1: tiles alternate gate / up (SwiGLU epilogue)
  float post = 1.0f;  // factor on every output: y = fp16((ascale * post) * acc)
  int cb = 0;  // 1: every zero is the codebook midpoint C/2 (the reference's canonical codebook)
  int ff = 0;  // 1: cb at 2 or 4 bits, so the folded integer path applies
  uint32_t* codes = nullptr;
  uint32_t* sz = nullptr;
  size_t bytes = 0;
};

// Pack one logical linear (row-major LSB-first codes, fp16 scale/zero
// [N][K/128]) into host buffers of the device layout.  For a gate/up pair
// call with both; columns are interleaved per 16-column tile.  xor8 is
// applied to 8-bit codes (0x80 for unsigned INT8 codes, 0 for signed int8).
void pack_linear_host(const uint8_t* codes, const uint16_t* scale, const uint16_t* zero, int N,
                      int K, int bits, uint32_t* out_codes, uint32_t* out_sz, int tile_stride,
                      int tile_offset, uint32_t xor8);

struct QGemmArgs {
  const int8_t* a;      // A tiles of [M][K]
  const float* as;      // [M] per-row activation scale
  const float* gs;      // [M][K/128] per-group code sums (float)
  uint16_t* out;        // [M][ldo]
  int32_t* tdump;       // optional [M][N][K/128]
  int M;
  int ldo;
  const int8_t* arow = nullptr;  // optional: the same codes row-major [M][K]
};
hipError_t launch_qgemm(const DLin& w, const QGemmArgs& a, hipStream_t st);
// One launch shape of the table (0..kQGemmVariants-1); all give identical
// bits.  Returns hipErrorInvalidValue where a shape does not apply.
constexpr int kQGemmVariants = 21;
hipError_t launch_qgemm_variant(const DLin& w, const QGemmArgs& a, int variant, hipStream_t st);

// FP16-activation dequant GEMM (qgemm_f16.hip): out = fp16(sum_k a * w) with
// w = (scale * alpha) * canonical codebook value, fp32 accumulation in
// ascending k (the weight rounded to fp16 for M > 1).  Codebook linears only.
struct F16Args {
  const uint16_t* a;      // fp16 [M][K], row-major
  const uint32_t* codes;  // a DLin's codes (not a gate/up pair)
  const uint32_t* sz;
  uint16_t* out;          // fp16 [M][N]
  int M, N, K, bits, nsteps, ng;
  float alpha;
};
hipError_t launch_qgemm_f16(const F16Args& p, hipStream_t st);

// Grouped-activation DPAS fold (qgemm_ga.hip): per 32-wide K op,
// acc += as(m, k0/ga) * ws * alpha * (2T - C S) * (1/C), out = fp16(acc).
struct GaArgs {
  const int8_t* a;        // int8 activations, A-tile layout (ceil(M/16)*16 rows)
  const float* as;        // fp32 [M][K / ga]
  const uint32_t* codes;  // a DLin's codes (not a gate/up pair)
  const uint32_t* sz;
  uint16_t* out;          // fp16 [M][N]
  int M, N, K, bits, nsteps, ng, ga;
  float alpha;
};
hipError_t launch_qgemm_ga(const GaArgs& p, hipStream_t st);

// ---- row kernels -----------------------------------------------------------
enum { SRC_X = 0, SRC_EMBED = 1, SRC_RESID = 2 };
struct RowQuantArgs {
  int src;                 // SRC_*
  const float* x;          // SRC_X: [M][K] fp32 input
  const float* embed;      // SRC_EMBED: [V][K]; tokens: [M]
  const int32_t* tokens;
  float* resid;            // SRC_EMBED: written; SRC_RESID: resid += rot?(y)
  const uint16_t* y;       // SRC_RESID: fp16 [M][K]
  int rot_y;               // SRC_RESID: rotate y before the add (left site)
  const int32_t* rowmap;   // optional: row m reads input row rowmap[m]
  const float* norm_w;     // optional RMSNorm(1+w)
  float eps;
  int rotate;              // FWHT the normed row (right site)
  int round;               // 0 half-away, 1 RNE
  int ga;                  // 0 per row, else slice width (64)
  int8_t* q;               // A tiles of [M][K]
  float* qscale;           // [M][K/ga or 1]
  float* gsum;             // optional [M][K/128]
  int M, K;
};
hipError_t launch_row_quant(const RowQuantArgs& a, hipStream_t st);

// Plain per-token quantization of an fp32 or fp16 [M][K] buffer (no norm, no
// rotation), K a multiple of 128 and <= kQuantPlainMaxK (a row held in the
// registers of one 256-thread workgroup, 8 values per thread per 2048).
constexpr int kQuantPlainMaxK = 20352;
hipError_t launch_quant_plain(const float* xf, const uint16_t* xh, int M, int K, int8_t* q,
                              float* qscale, float* gsum, hipStream_t st);

// ---- q/k norm + RoPE + KV append --------------------------------------------
// KV pages: one 32-token x 128-dim block per (page, kv_head), stored in the
// order the attention MFMAs consume it, so each wave load is one contiguous
// run of 64 lanes x 8 elements:
//   K: fragment (h = t % 2, i = d / 32), lane 16 * ((d / 8) % 4) + t / 2,
//      element d % 8   (S^T = K Q^T: A-operand rows are tokens 2c + h)
//   V: fragment (d / 16), lane 16 * (t / 8) + d % 16, element t % 8
//      (O^T = V^T P^T: A-operand rows are dims, k runs over tokens)
// Index of token t, dim d inside its block of 32 * 128 elements:
__host__ __device__ inline int kv_koff(int t, int d) {
  return ((((t & 1) * 4 + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 + (t >> 1)) << 3) + (d & 7);
}
__host__ __device__ inline int kv_voff(int t, int d) {
  return (((d >> 4) * 64 + (t >> 3) * 16 + (d & 15)) << 3) + (t & 7);
}
struct KVLayout {
  int nkv, hd, page;          // page = tokens per page (32); hd = 128
  int max_pages;              // block-table row length
  int kv_int8;
  void* kpool;                // this layer: [pages][nkv][32 * 128] (fp16 or int8), kv_koff order
  void* vpool;                // this layer: [pages][nkv][32 * 128], kv_voff order
  uint16_t* kscale;           // int8: [pages][nkv][page] fp16
  uint16_t* vscale;
  const int32_t* block_table; // [max_seqs][max_pages]
};
struct QKArgs {
  const uint16_t* qkv;        // [M][nqb*hd + 2*nkv*hd] fp16, nqb = nq (2 nq gated)
  const int32_t* row_seq;     // [M]
  const int32_t* row_pos;     // [M]
  const float* q_norm;        // [hd] or null
  const float* k_norm;
  const float* rope_cos;      // [max_pos][rotary/2]
  const float* rope_sin;
  int rotary;
  float eps;
  int nq;
  uint16_t* qout;             // [M][nq][hd] fp16
  int M;
  // 1: the q heads of the QKV output are [q | gate] pairs (head-sized column
  // block 2h is q head h, 2h + 1 its gate), and the gate is copied, as the
  // fp16 GEMM output, to gout [M][nq][hd]
  int gated;
  uint16_t* gout;
};
// Head-sized column block b of the QKV output: its kind (0 q, 1 k, 2 v,
// 3 gate) and head index within that kind.
__host__ __device__ inline void qkv_block(int b, int nq, int nkv, int gated, int& kind, int& hh) {
  const int nqb = gated ? 2 * nq : nq;
  if (b < nqb) {
    kind = gated && (b & 1) ? 3 : 0;
    hh = gated ? b >> 1 : b;
  } else if (b < nqb + nkv) {
    kind = 1;
    hh = b - nqb;
  } else {
    kind = 2;
    hh = b - nqb - nkv;
  }
}
hipError_t launch_qk_rope_kv(const QKArgs& a, const KVLayout& kv, hipStream_t st);
// The QKV projection with the q/k norm + RoPE + KV append as its epilogue
// (launch_qgemm followed by launch_qk_rope_kv, bit-identical, without the
// fp16 QKV buffer).  variant < 0: the default launch shape.  Returns
// hipErrorInvalidValue where that shape is not a one-head-per-workgroup row
// block (then run the two passes).
hipError_t launch_qgemm_qkrope(const DLin& w, const QGemmArgs& a, const QKArgs& qa, const KVLayout& kv, int variant,
                               hipStream_t st);

// ---- KV page copy (prefix reuse) ----------------------------------------------
// Copies n pages, sp[i] -> dp[i] (device page indices), in each of npools
// pools; pools[j] is a device pool whose pages are page_bytes[j % per]
// bytes (per = pools per layer: K, V [, K scales, V scales]).
struct PageCopyArgs {
  void* const* pools;        // device array [npools]
  int npools, per;
  size_t page_bytes[4];      // multiples of 16
  const int32_t* sp;
  const int32_t* dp;
  int n;
};
hipError_t launch_copy_pages(const PageCopyArgs& a, hipStream_t st);

// ---- ragged batch packing ---------------------------------------------------
struct AttnUnit {
  int seq, kvh, row0, qn, qpos0, kv_lo, kv_hi, pad;
};
struct PackOut {
  int32_t* cu_seqlens;   // [ngroups + 1]
  int32_t* row_grp;      // [M]
  int32_t* row_seq;      // [M]
  int32_t* row_pos;      // [M]
  int32_t* row_kind;     // [M]
  int32_t* comb_base;    // [M] unit index of (q-block, kvh 0, split 0)
  int32_t* comb_nsplit;  // [M]
  int32_t* comb_tok;     // [M] token index inside its q-block
  AttnUnit* units;       // [n_units]
  int32_t* want_rows;    // [n_want] rows to score, in row order
  int32_t* order;        // [n_slots] attention dispatch slot -> unit (-1: idle)
  int32_t* row_tok = nullptr;  // [M] the rows' token ids (optional)
};
// Attention dispatch order (4 slots = the 4 waves of one workgroup).  A
// sequence group with several q-blocks is cut into chunks of 4 consecutive
// q-blocks; for each (chunk, kv head, split) its 4 q-blocks take the 4 waves
// of one workgroup, so they stream the same K/V pages together (one wave
// idles where a q-block has no such split).  Groups with one q-block (decode
// rows) follow, their units packed densely.  The host count of the slots;
// *chunked receives the size of the chunked region (a multiple of 4).
long attn_slot_count(const int* g_pos0, const int* g_len, int ngroups, int nkv, int split, int qb,
                     long* chunked = nullptr);
// rows: device copy of ifr_row[M] (5 int32 each).  qb = q-block tokens,
// split = kv tokens per unit (multiple of the page size).
hipError_t launch_pack(const int32_t* rows, int M, int nkv, int qb, int split, const PackOut& o,
                       hipStream_t st);

// ---- attention ------------------------------------------------------------------
struct AttnArgs {
  const AttnUnit* units;
  int n_units;
  const int32_t* order;    // [n_slots] dispatch slot -> unit or -1
  int n_slots;
  int n_shared;            // slots [0, n_shared): chunked workgroups that share K/V pages in LDS
  const uint16_t* q;       // [M][nq][hd]
  int nq;
  float scale_log2;        // log2(e) / sqrt(hd)
  float* part_o;           // [n_units][16 * col_tiles][hd]
  float* part_ml;          // [n_units][16 * col_tiles][2]
  int col_tiles;           // 16-column MFMA tiles per unit (1 or 2): q-block = 16 * col_tiles / G tokens
};
hipError_t launch_attention(const AttnArgs& a, const KVLayout& kv, hipStream_t st);

struct CombineArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* comb_base;
  const int32_t* comb_nsplit;
  const int32_t* comb_tok;
  int M, nq, nkv, hd;
  float* attn_out;         // optional fp32 [M][nq*hd]
  int8_t* q;               // A tiles of [M][nq*hd], per-token int8 (half-away)
  float* qscale;           // [M]
  float* gsum;             // [M][nq*hd/128]
  int ucols;               // partial columns per unit (16 * col_tiles)
  // optional fp16 [M][nq*hd] attention output gate: the merged row is scaled
  // by sigmoid(gate) = 1 / (1 + exp(-gate)) before it is quantized
  const uint16_t* gate;
};
hipError_t launch_combine(const CombineArgs& a, hipStream_t st);

// ---- lm_head + argmax ---------------------------------------------------------
struct LmHeadArgs {
  const int8_t* a;         // [W][H] GA64 RNE codes
  const float* as;         // [W][H/64]
  const uint32_t* wcodes;  // int8 weights in the bits=8 fragment layout
  const uint16_t* wscale;  // [V] fp16 per-row scale
  int W, V, H;
  float* logits;           // optional [W][V]
  float* part_val;         // [nparts][W]
  int32_t* part_idx;
  int32_t* best;           // [W]
  int nparts;              // filled by the launcher
};
int lmhead_nparts(int V);
hipError_t launch_lmhead(LmHeadArgs& a, hipStream_t st);

// mg = fp16(silu(g) * u) over an unpaired [M][2F] gate|up fp16 buffer.
hipError_t launch_swiglu(const uint16_t* gu, int M, int F, uint16_t* mg, hipStream_t st);

// Gather rows for scoring: dst[i] = src[rows[i]] over H floats.
hipError_t launch_gather_rows(const float* src, const int32_t* rows, int n, int H, float* dst,
                              hipStream_t st);

}  // namespace ifrk
