/*
 * intfer_amd.h -- C-ABI of the MI355X-native mixed-batch M-row forward.
 *
 * The reference drives its device layer through a C++ virtual interface
 * (`struct LinearBackend`, examples/intfer_cli/main.cpp:455-566) and the
 * `intfer::Engine` below it (include/intfer/engine.hpp:37-562).  This header
 * replaces both with plain-C entry points: POD arguments, opaque handles,
 * int status codes, no exceptions, no torch or HIP types in any signature.
 *
 * Threading: a context is single-threaded, like the reference's one
 * dispatcher thread (main.cpp:9394-9402).  All device work of a context runs
 * in order on the context's one HIP stream.
 *
 * Errors: every entry point returns IFR_OK or a negative IFR_E* code;
 * ifr_last_error() returns a message for the last failure on this thread.
 * IFR_EDECLINE keeps the reference's "decline, caller runs its host path"
 * meaning (engine.hpp:102-118): nothing was written.
 */
#ifndef INTFER_AMD_H
#define INTFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  IFR_OK = 0,
  IFR_EDECLINE = -1, /* shape/format not handled: caller keeps its own path */
  IFR_EINVAL = -2,   /* bad argument */
  IFR_ENOMEM = -3,   /* device or host allocation failed / pool exhausted */
  IFR_EDEVICE = -4,  /* HIP runtime error, or no device */
  IFR_ESTATE = -5    /* call not valid in the current context state */
};

/* ------------------------------------------------------------------------
 * Model description (host side).
 * ---------------------------------------------------------------------- */

/* Decoder configuration.  Mirrors the fields of the reference ModelConfig
 * that the full-attention layer reads (main.cpp:91-132).  The synthetic
 * 0.8B-class model is hidden 1024, 28 layers, 16 q / 8 kv heads, head_dim
 * 128, SwiGLU 3072, vocab 151936, eps 1e-6, theta 1e6, rotary_dim 128. */
typedef struct ifr_model_cfg {
  int32_t hidden;
  int32_t layers;
  int32_t n_heads;
  int32_t n_kv;
  int32_t head_dim;
  int32_t inter;
  int32_t vocab;
  int32_t rotary_dim;
  float rms_eps;
  float rope_theta;
  int32_t group_size; /* weight K-group (128) */
  int32_t qk_norm;    /* 1: per-head RMSNorm(1+w) on q and k (main.cpp:7641-7650) */
  int32_t rotate;     /* 1: online Hadamard at the QKV/O/FFN_IN/FFN_OUT sites */
  int32_t attn_gate;  /* 1: attention output gate (ModelConfig::attn_output_gate,
                       * main.cpp:108): q_proj has 2 * n_heads * head_dim rows,
                       * head h's q rows [2h*hd, 2h*hd + hd) followed by its gate
                       * rows [2h*hd + hd, 2h*hd + 2hd) (main.cpp:7625-7640), and
                       * the attention output is scaled by sigmoid(gate) before
                       * the O projection (:7697-7698); 0: q_proj has
                       * n_heads * head_dim rows, no gate */
  int32_t attn_gate_off; /* 1: a packed q_proj (attn_gate = 1) keeps its layout
                          * but the gate is not applied, as the reference does
                          * when config.json sets attn_output_gate false
                          * (main.cpp:250, :7697: the sigmoid needs both
                          * packed_gate and the flag); 0 (default, the
                          * reference's default true): applied */
} ifr_model_cfg;

/* One quantized linear y = W x, W is [N][K].  Logical (load) layout:
 *   codes : row-major packed, least-significant bits first: code(n,k) is
 *           bits [(i*b)%8, +b) of byte (i*b)/8 with i = n*K + k (the
 *           reference packing, src/quant/dashq.cpp:387-402, applied row-major)
 *   scale : fp16 [N][K/group]
 *   zero  : fp16 [N][K/group]
 *   post  : fp32 factor on every output of the linear (0 is read as 1)
 * Dequantized weight: w(n,k) = post * scale(n,g) * (code(n,k) - zero(n,g)),
 * g = k/group.  The reference codebook (dashq.cpp:405-417, (2c-C)/C with
 * C = 2^b - 1) scaled by s_g * alpha (dashq.cpp:531-575) is the special case
 * scale = s_g, zero = C/2, post = 2*alpha/C: every factor is stored exactly. */
typedef struct ifr_linear {
  int32_t N, K, bits, group;
  const uint8_t* codes;
  const uint16_t* scale;
  const uint16_t* zero;
  float post;
} ifr_linear;

typedef struct ifr_layer_w {
  ifr_linear q, k, v, o, gate, up, down;
  const float* in_ln;   /* [hidden]  RMSNorm(1+w) before attention */
  const float* post_ln; /* [hidden]  RMSNorm(1+w) before the MLP */
  const float* q_norm;  /* [head_dim] */
  const float* k_norm;  /* [head_dim] */
} ifr_layer_w;

typedef struct ifr_host_model {
  ifr_model_cfg cfg;
  const float* embed;      /* [vocab][hidden] fp32 */
  const float* final_norm; /* [hidden] */
  const ifr_layer_w* layers; /* [layers] */
  const float* lm_head;    /* [vocab][hidden] untied output projection; NULL:
                            * tied with embed (the 0.8B case, main.cpp:8302-8307) */
} ifr_host_model;

/* Synthetic seeded model (portable splitmix64 + Box-Muller; see the
 * generator source for distributions).  bits_mode 2 or 4 = every linear at
 * that width; bits_mode 0 = seeded per-tensor 70 % INT2 / 30 % INT4 split.
 * OR-ing IFR_SYNTH_INTFER into bits_mode draws the weights in the form the
 * .intfer container stores exactly: one fp16 scale per K-group shared by
 * all rows, zero = C/2, post = 2/C, embedding and norms rounded to fp16.
 * The returned model owns its buffers; free with ifr_host_model_free. */
#define IFR_SYNTH_INTFER 0x100
ifr_host_model* ifr_synth_model(const ifr_model_cfg* cfg, uint64_t seed, int32_t bits_mode);
/* Frees a model returned by ifr_synth_model or ifr_intfer_host_model. */
void ifr_host_model_free(ifr_host_model* m);
void ifr_synth_free(ifr_host_model* m); /* same as ifr_host_model_free */

/* Default 0.8B-class configuration. */
void ifr_default_cfg(ifr_model_cfg* out);

/* ------------------------------------------------------------------------
 * Context, memory helpers.
 * ---------------------------------------------------------------------- */
typedef struct ifr_ctx ifr_ctx;

const char* ifr_last_error(void);
/* Replaces Engine::load + DeviceManager::discover (engine.cpp:552,
 * device_manager.cpp:30).  One HIP stream per context. */
int ifr_ctx_create(int32_t device, ifr_ctx** out);
int ifr_ctx_destroy(ifr_ctx* ctx);
int ifr_sync(ifr_ctx* ctx);
/* No reference counterpart: the context's HIP stream (a hipStream_t), for
 * callers that order their own work or timing events against the engine. */
void* ifr_ctx_stream(ifr_ctx* ctx);
/* No reference counterpart: HIP events on the context stream around any
 * work enqueued between the two calls (bench hook).  ifr_timer_end waits for
 * the end event and returns the elapsed device time in milliseconds. */
int ifr_timer_begin(ifr_ctx* ctx);
int ifr_timer_end(ifr_ctx* ctx, double* ms);

/* No reference counterpart: measured peaks of the device, the denominators
 * reported next to the nominal ones.  ifr_peak_read streams `bytes` (at
 * least 1 GiB, above the 256 MB Infinity Cache; a multiple of 16) from buf_d
 * once per launch, `reps` launches timed with HIP events on the context
 * stream, and returns the read bandwidth in GB/s.  ifr_peak_mfma runs
 * back-to-back independent MFMAs in two waves per SIMD, `iters` rounds of 8
 * per wave: dtype 0 v_mfma_i32_16x16x64_i8 (int8 ops), 1
 * v_mfma_f32_16x16x32_f16 (fp16 flops); returns TOP/s (TFLOP/s). */
int ifr_peak_read(ifr_ctx* ctx, const void* buf_d, size_t bytes, int32_t reps, double* gbps);
int ifr_peak_mfma(ifr_ctx* ctx, int32_t dtype, int32_t iters, int32_t reps, double* tops);

/* Device buffers for tests and benches (no torch in the boundary). */
int ifr_malloc(ifr_ctx* ctx, size_t bytes, void** dptr);
int ifr_free(ifr_ctx* ctx, void* dptr);
int ifr_h2d(ifr_ctx* ctx, void* dst, const void* src, size_t bytes);
int ifr_d2h(ifr_ctx* ctx, void* dst, const void* src, size_t bytes);
int ifr_memset(ifr_ctx* ctx, void* dst, int value, size_t bytes);
/* Device-to-device copy, enqueued on the context stream (not waited for);
 * also the known-size copy that calibrates HBM traffic counters. */
int ifr_d2d(ifr_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ------------------------------------------------------------------------
 * Kernel-level entry points (tests, benches, and the reference's
 * free kernel functions, include/intfer/gemm/quant_gemm.hpp).
 * All pointers named *_d are device pointers.
 * ---------------------------------------------------------------------- */

/* A quantized linear repacked to the device MFMA layout.  Replaces
 * Engine::shard_weight + repack_dpas412 (engine.cpp:434-549,
 * quant_gemm.cpp:3294-3322). */
typedef struct ifr_dlinear ifr_dlinear;
int ifr_linear_upload(ifr_ctx* ctx, const ifr_linear* w, ifr_dlinear** out);
int ifr_linear_free(ifr_ctx* ctx, ifr_dlinear* w);
/* Bytes of the device copy (codes + scale/zero), for roofline accounting. */
size_t ifr_linear_bytes(const ifr_dlinear* w);

/* Int8 GEMM activations ("A tiles"): 16 rows x 64 columns per 1 KB tile,
 * tiles ordered (row block, column block); inside a tile the 16 bytes one
 * MFMA lane consumes are contiguous, so a wavefront reads a 16 x 64 operand
 * with one coalesced 1 KB load.  Element (m, k) of an [M][K] matrix sits at
 * byte IFR_ATILE_OFF(m, k, K); a buffer holds ceil(M/16)*16*K bytes (the
 * padding rows are never read into an output). */
#define IFR_ATILE_OFF(m, k, K)                                                   \
  ((((size_t)(m) >> 4) * ((size_t)(K) >> 6) + ((size_t)(k) >> 6)) * 1024 +      \
   ((((size_t)(k) & 63) >> 4) * 16 + ((size_t)(m) & 15)) * 16 + ((size_t)(k) & 15))

/* Per-token int8 activation quantization with optional fused pre-ops.
 * Replaces dashq::act_quant_ga64_batch / act_quant_ga64_dev
 * (dashq.cpp:221-336, quant_gemm.cpp:3325-3392) for a per-row (GA = K)
 * or GA = 64 slice.  x_d fp32 [M][K].  Outputs: q_d int8 [M][K] in the
 * A-tile layout (IFR_ATILE_OFF below; ceil(M/16)*16*K bytes),
 * scale_d fp32 [M][K/ga], gsum_d fp32 [M][K/128] (sum of the int8 codes
 * per 128-column group; may be NULL).
 *   norm_w_d : if non-NULL, x is first replaced by RMSNorm(1+w)(x) (main.cpp:337-351)
 *   rotate   : if 1, then x <- FWHT(x)/sqrt(K) (spinquant.cpp:586-604)
 *   round    : 0 half-away-from-zero (trunk), 1 nearest-even (lm_head)
 *   ga       : 0 = per row, else slice width (64) */
int ifr_act_quant(ifr_ctx* ctx, const float* x_d, int32_t M, int32_t K,
                  const float* norm_w_d, float eps, int32_t rotate, int32_t round,
                  int32_t ga, int8_t* q_d, float* scale_d, float* gsum_d);

/* W2A8 / W4A8 / W8A8 GEMM with int32 accumulation (replaces
 * quant_gemm_dpas48 / dpas48_tiled, quant_gemm.cpp:3492-3791):
 *   T(m,n,g) = sum_{k in g} a_q(m,k) * code(n,k)            (int32, exact)
 *   S(m,g)   = sum_{k in g} a_q(m,k)                         (gsum_d)
 *   acc(m,n) = fold over g ascending of
 *                d = fma(-zero(n,g), S(m,g), T(m,n,g)); acc = fma(scale(n,g), d, acc)
 *   y(m,n)   = fp16_rne((ascale(m) * post) * acc(m,n))
 * a_d holds the int8 activations in the A-tile layout (IFR_ATILE_OFF), as
 * ifr_act_quant writes them.  out_d fp16 [M][N].  tdump_d, if non-NULL,
 * receives T as int32 [M][N][K/128]. */
int ifr_quant_gemm(ifr_ctx* ctx, const ifr_dlinear* w, const int8_t* a_d,
                   const float* ascale_d, const float* gsum_d, int32_t M,
                   uint16_t* out_d, int32_t* tdump_d);

/* Same GEMM over the interleaved [gate;up] pair with the SwiGLU epilogue
 * mg = fp16(silu(g) * u), g,u the fp16 GEMM outputs (main.cpp:7754-7758,
 * silumul_to_half quant_gemm.cpp:4209).  out_d fp16 [M][N_gate]. */
int ifr_linear_upload_pair(ifr_ctx* ctx, const ifr_linear* gate, const ifr_linear* up,
                           ifr_dlinear** out);
int ifr_quant_gemm_swiglu(ifr_ctx* ctx, const ifr_dlinear* gate_up, const int8_t* a_d,
                          const float* ascale_d, const float* gsum_d, int32_t M,
                          uint16_t* out_d);

/* No counterpart in the reference (its DPAS kernels have one fixed shape):
 * run ifr_quant_gemm / ifr_quant_gemm_swiglu with launch shape `variant`
 * (0 .. ifr_quant_gemm_variants()-1) instead of the size heuristic, for
 * parity tests and tuning.  Every shape yields identical bits; IFR_EDECLINE
 * where a shape does not apply to (M, N, K). */
int ifr_quant_gemm_variants(void);
int ifr_quant_gemm_variant(ifr_ctx* ctx, const ifr_dlinear* w, const int8_t* a_d,
                           const float* ascale_d, const float* gsum_d, int32_t M,
                           uint16_t* out_d, int32_t variant);

/* No counterpart in the reference (its activation codes have one layout):
 * ifr_quant_gemm (plain linear) or ifr_quant_gemm_swiglu (gate/up pair) with
 * the activation codes also given row-major, arow_d int8 [M][K] (the codes of
 * a_d's M rows, unpadded).  The decode weight stream (M <= 4, K >= 4096)
 * stages its A rows from arow_d, K contiguous bytes per row, where in the
 * A-tile layout a row holds 16 of every 128 bytes it touches; every other
 * launch shape reads a_d.  arow_d may be NULL.  variant: -1 for the size
 * heuristic, else a launch shape as in ifr_quant_gemm_variant (IFR_EDECLINE
 * where it does not apply).  The bits are those of ifr_quant_gemm. */
int ifr_quant_gemm_rows(ifr_ctx* ctx, const ifr_dlinear* w, const int8_t* a_d,
                        const int8_t* arow_d, const float* ascale_d, const float* gsum_d,
                        int32_t M, uint16_t* out_d, int32_t variant);

/* FP16-activation dequant GEMM (replaces quant_gemm_forward_usm, the
 * reference's default GPU linear, quant_gemm.cpp:359-2153):
 *   out(m,n) = fp16_rne( sum_k a(m,k) * w(n,k) ), fp32, k ascending
 *   w(n,k)   = (scale(n,k/128) * alpha) * cb(code(n,k)),
 * cb the canonical codebook (2c - C)/C as fp32 ({-1, -1/3, 1/3, 1} for
 * INT2; canon_value :139-144).  M == 1 keeps w in fp32 and accumulates
 * acc = fma(a, w, acc) (the decode kernels :1026-1080, :2022-2066); M > 1
 * rounds w to fp16 as the tiled kernel stages it (:2069-2150).  a_d fp16
 * [M][K] row-major, out_d fp16 [M][N]; alpha is the tensor's global factor
 * (1 when it has none).  IFR_EDECLINE for a gate/up pair, a linear whose
 * zeros are not all C/2 (the reference path knows only the codebook), or
 * K > 32768 at M == 1. */
int ifr_quant_gemm_f16(ifr_ctx* ctx, const ifr_dlinear* w, const uint16_t* a_d, int32_t M,
                       float alpha, uint16_t* out_d);

/* W2A8 / W4A8 / W8A8 GEMM with grouped activation scales: the reference's
 * DPAS fold as written (dpas48_tiled, quant_gemm.cpp:3492-3791; per-op math
 * :3602-3736; act_group GA, As[r][k0/GA] :3502, :3614; Dpas48Params
 * quant_gemm.hpp:522-558).  For each 32-wide K op o, ascending (k0 = 32 o):
 *   T = sum a_q(m,k) c(n,k),  S = sum a_q(m,k)            (int32, exact)
 *   acc += as(m, k0/ga) * ws(n, k0/128) * alpha * (2T - C S) * (1/C)
 *   out(m,n) = fp16_rne(acc)
 * left to right in fp32, each product and the add rounded (no contraction:
 * the reference's device compiler may fuse the last step, which this does
 * not).  a_d: int8 activations in the A-tile layout (IFR_ATILE_OFF), as
 * ifr_act_quant writes them with the same ga; ascale_d fp32 [M][K/ga];
 * ga a multiple of 64 dividing K (64 the reference's default, 0 = K: one
 * scale per row); out_d fp16 [M][N].  IFR_EDECLINE for a gate/up pair or a
 * linear whose zeros are not all C/2 (the fold has no zero term). */
int ifr_quant_gemm_ga(ifr_ctx* ctx, const ifr_dlinear* w, const int8_t* a_d, const float* ascale_d,
                      int32_t M, int32_t ga, float alpha, uint16_t* out_d);

/* ------------------------------------------------------------------------
 * Engine: model load, paged KV, one mixed iteration.
 * ---------------------------------------------------------------------- */
typedef struct ifr_kv_cfg {
  int32_t max_seqs;       /* sequence slots */
  int32_t max_seq_tokens; /* per-sequence KV capacity (INTFER_KV_CAP analogue, main.cpp:4348-4361) */
  int32_t pool_tokens;    /* total KV tokens in the page pool */
  int32_t kv_int8;        /* 0 fp16 KV; 1 int8 KV with fp16 scale per (token, kv_head) */
  int32_t max_rows;       /* largest M one ifr_forward call may carry */
  int32_t attn_split;     /* KV tokens per attention work unit, a multiple of 32
                           * (0: 256).  Fixed per engine, so a row's attention
                           * never depends on the rest of the batch. */
  int32_t lanes;          /* concurrent sub-batches per forward on the
                           * context's streams: 1 or 2 (0: 1).  Two lanes
                           * measured no faster on the serve load: each layer
                           * is a chain of latency-bound kernels whose time
                           * barely shrinks with half the rows. */
  int32_t separate_qk;    /* 0: the q/k norm + RoPE + KV append runs as the
                           * QKV GEMM's epilogue where the launch shape is one
                           * head per workgroup (bit-identical); 1: always as
                           * its own pass */
  int32_t dense_attention; /* 0: the q-blocks of a prefill chunk that share a
                            * kv head and KV split run in one workgroup that
                            * copies each K/V page once into LDS for all of
                            * them (fp16 KV); 1: every attention unit runs on
                            * its own (bit-identical; a check of the first) */
} ifr_kv_cfg;

/* Upload + repack a model (replaces Engine::load, build_shards,
 * preload_all, engine.cpp:552-743, :1071).  The host model may be freed
 * afterwards. */
int ifr_model_load(ifr_ctx* ctx, const ifr_host_model* m, const ifr_kv_cfg* kv);

/* No reference counterpart: the configuration of the loaded model. */
int ifr_model_info(ifr_ctx* ctx, ifr_model_cfg* out);

/* Sequence slots over the paged KV pool.  truncate = speculative rollback
 * (main.cpp:11896-11915) and prefix reuse: KV beyond len is dropped. */
int ifr_seq_open(ifr_ctx* ctx, int32_t* slot);
int ifr_seq_close(ifr_ctx* ctx, int32_t slot);
int ifr_seq_truncate(ifr_ctx* ctx, int32_t slot, int32_t len);
int ifr_seq_len(ifr_ctx* ctx, int32_t slot, int32_t* len);
/* Per-sequence KV capacity in tokens of the loaded model. */
int ifr_kv_capacity(ifr_ctx* ctx, int32_t* tokens);
/* Fill the empty sequence dst with the first len cached positions of src
 * (a device page copy; every layer, K, V and int8 scales).  Replaces the
 * prefix cache's host KV snapshot restore (PrefixCache::install,
 * main.cpp:9614-9680): the KV of a position depends only on the tokens up
 * to it, so the copy equals what prefilling that prefix would append. */
int ifr_seq_copy_prefix(ifr_ctx* ctx, int32_t dst, int32_t src, int32_t len);
/* Fill an open, empty sequence with len cached positions: k, v are fp32
 * host arrays [layers][len][n_kv][head_dim]; values are stored exactly as
 * the forward stores them (fp16 round, or int8 with an fp16 scale per
 * (token, kv_head)).  Used for the configs' seeded cached contexts. */
int ifr_seq_load_kv(ifr_ctx* ctx, int32_t slot, int32_t len, const float* k, const float* v);

/* ------------------------------------------------------------------------
 * Per-linear seam over the loaded model: the reference's LinearBackend
 * (main.cpp:455-566), for a caller that keeps its own forward (step_batch)
 * and hands the device one linear at a time.  Host fp32 rows in, host fp32
 * rows out, as the reference's GPU backend returns them (half_to_float of
 * the device's fp16 outputs, dashq.cpp:111).  The linear runs the forward's
 * integer contract: per-token int8 quantization of each input row
 * (half-away, s = max|x| / 127, dashq.cpp:221-336), int32 T, the fp32 group
 * fold, fp16 output (ifr_quant_gemm).  Inputs are taken as the caller
 * passes them: the SpinQuant rotation of a site is the caller's (rot_for,
 * main.cpp:436-445; ifr_linear_rot says which applies).  Rows are
 * independent, so any M gives each row the bits it has alone.
 * ---------------------------------------------------------------------- */
enum {
  IFR_LIN_Q = 0, IFR_LIN_K = 1, IFR_LIN_V = 2, IFR_LIN_O = 3,
  IFR_LIN_GATE = 4, IFR_LIN_UP = 5, IFR_LIN_DOWN = 6
};
/* The reference's tensor names ("model.language_model.layers.<l>.
 * self_attn.q_proj.weight", ...; main.cpp:4225-4270) to (layer, IFR_LIN_*).
 * IFR_EINVAL for a name that is not one of the loaded model's linears. */
int ifr_linear_lookup(ifr_ctx* ctx, const char* tensor_name, int32_t* layer, int32_t* which);
/* Shape (N rows, K columns) of a linear; Q of a gated model is the packed
 * [q, gate] projection of 2 * n_heads * head_dim rows, as the file holds it. */
int ifr_linear_shape(ifr_ctx* ctx, int32_t layer, int32_t which, int32_t* N, int32_t* K);
/* LinearBackend::rot_for (main.cpp:436-445): 0 no rotation, 1 the right
 * site (FWHT of the input: q, k, v, gate, up), 2 the left site (FWHT of the
 * output: o, down); the rotation is the canonical Sylvester Hadamard the
 * loader accepts (spinquant.cpp:586-604). */
int ifr_linear_rot(ifr_ctx* ctx, int32_t which, int32_t* site);
/* LinearBackend::run_linear_batch (main.cpp:474-488): Y[M][N] = W X for host
 * X[M][K]. */
int ifr_linear_batch(ifr_ctx* ctx, int32_t layer, int32_t which, const float* X, float* Y, int32_t M);
/* LinearBackend::run_linear_wave_batch (main.cpp:514-527): independent
 * linears over M rows each (no item's Y may alias another's X or Y), one
 * device round trip for all of them; each Y equals its ifr_linear_batch. */
typedef struct ifr_linear_item {
  int32_t layer, which;
  const float* X;  /* [M][K] */
  float* Y;        /* [M][N] */
} ifr_linear_item;
int ifr_linear_wave_batch(ifr_ctx* ctx, const ifr_linear_item* items, int32_t n, int32_t M);
/* LinearBackend::run_mlp_fused (main.cpp:528-540): md[M][hidden] =
 * W_down (silu(W_gate rin) * (W_up rin)) on the device, for host rin[M][hidden]
 * (the normed, right-rotated MLP input); the left rotation of md stays the
 * caller's.  silu(g) * u is formed from the fp16 gate and up outputs and
 * rounded to fp16 (silumul_to_half, quant_gemm.cpp:4209), then quantized
 * per token for the down projection, as the forward does. */
int ifr_mlp_fused(ifr_ctx* ctx, int32_t layer, const float* rin, float* md, int32_t M);

enum { IFR_ROW_DECODE = 0, IFR_ROW_PREFILL = 1, IFR_ROW_VERIFY = 2 };

/* One row of the ragged batch (BatchItem, main.cpp:4831, extended with the
 * verify kind).  Rows of one sequence must be contiguous with consecutive
 * positions starting at that sequence's current KV length. */
typedef struct ifr_row {
  int32_t seq;   /* sequence slot */
  int32_t pos;   /* absolute position of this row's token */
  int32_t token; /* input token id */
  int32_t kind;  /* IFR_ROW_* */
  int32_t want;  /* 0: not scored; 1: scored (argmax); 2: scored, and its
                  * logits returned (rows the caller samples from) */
} ifr_row;

/* One mixed iteration (replaces step_batch main.cpp:7519-8320 and the
 * LinearBackend calls it makes).  best_out[M]: argmax (first max wins) for
 * scored rows (want >= 1), -1 otherwise.  logits_out, if non-NULL, receives
 * fp32 [n][vocab] logits in row order: of the rows with want = 2 when there
 * are any, else of every scored row.  The call appends every row's K/V to
 * its sequence. */
int ifr_forward(ifr_ctx* ctx, const ifr_row* rows, int32_t M, int32_t* best_out,
                float* logits_out);

/* Ragged joint attention alone over the resident KV of `layer` (kernel-level
 * entry; replaces the host attention loop, main.cpp:7657-7701, and the
 * demo flash kernels, src/attention/flash_attention.cpp:30-273).  Rows as in
 * ifr_forward but their KV must already be present (pos < sequence length);
 * nothing is appended.  q_h: fp16 bits [M][n_heads][head_dim]; out_h: fp32
 * [M][n_heads*head_dim]. */
int ifr_attention(ifr_ctx* ctx, int32_t layer, const ifr_row* rows, int32_t M,
                  const uint16_t* q_h, float* out_h);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ifr_attention with device buffers q_d (fp16 bits
 * [M][n_heads][head_dim]) and out_d (fp32 [M][n_heads*head_dim]), and every
 * intermediate (row maps, attention units, split-KV partials, the combine's
 * int8 codes) in a fixed per-GPU device array of the library (about 37 MB,
 * held by each GPU the library runs on until the process ends).  The call
 * makes no hipMalloc / hipFree.  Limits: M <= 512 rows, n_heads * head_dim <=
 * 8192, and at most 4096 attention units (one per q-block of 16 / GQA-group
 * tokens, kv head and 256-token KV split); beyond them it returns IFR_EINVAL
 * with a message and does nothing.  Results are bit-identical to
 * ifr_attention's.  Every call on one GPU shares that array, so calls on one
 * GPU from other threads or contexts of the process wait for each other (a
 * per-device lock held from the first launch until out_d is written); each
 * process has its own array.  Returns after out_d is written. */
int ifr_attention_noalloc(ifr_ctx* ctx, int32_t layer, const ifr_row* rows, int32_t M,
                          const uint16_t* q_d, float* out_d);

/* Per-kernel device timing of ifr_forward calls since ifr_set_timing(ctx, 1)
 * (HIP events on the launching stream; while it is on, every forward runs
 * on one stream so each kernel is timed alone), for the bench.  Names:
 * "qgemm_qkv", "qgemm_o", "qgemm_gate_up", "qgemm_down", "attention",
 * "combine", "row_quant", "quant_plain", "qk_rope_kv", "lmhead", "pack".
 * bytes / flops accumulate each launch's algorithmic HBM bytes and
 * arithmetic work (int8 ops for the GEMMs, fp flops for attention).
 * "host_submit" / "host_wait" (host milliseconds of each forward spent
 * enqueuing, then waiting for the device) accumulate on every forward, the
 * counterpart of the reference engine's submit / waitblock buckets
 * (include/intfer/engine.hpp:567-630); ifr_set_timing clears them. */
int ifr_set_timing(ifr_ctx* ctx, int32_t on);
int ifr_get_timing(ifr_ctx* ctx, const char* kernel, double* total_ms, int64_t* launches,
                   double* bytes, double* flops);

/* Test hook (no reference counterpart): copies the last forward's packing
 * outputs to host buffers (any may be NULL).  units: 8 int32 per unit
 * {seq, kv_head, row0, q_tokens, q_pos0, kv_lo, kv_hi, 0}. */
int ifr_debug_pack(ifr_ctx* ctx, int32_t M, int32_t* cu_seqlens, int32_t* row_grp,
                   int32_t* comb_base, int32_t* comb_nsplit, int32_t* comb_tok, int32_t* units,
                   int32_t* n_units, int32_t* split);
/* Test hook (no reference counterpart): the last forward's attention
 * dispatch order (slot -> unit index, -1 idle; 4 slots per workgroup) into
 * order[0..cap); *n_slots receives its length. */
int ifr_debug_attn_order(ifr_ctx* ctx, int32_t* order, int32_t cap, int32_t* n_slots);
/* Test hook (no reference counterpart): how many sub-batches (1 or 2) the
 * last ifr_forward ran concurrently on the context's two streams.  A batch
 * is cut into [decode / verify rows | prefill chunks], or decode rows are
 * halved by KV length; while per-kernel timing is on, every batch runs as one. */
int ifr_debug_last_lanes(ifr_ctx* ctx, int32_t* lanes);

/* ------------------------------------------------------------------------
 * .intfer model files (the INTFER1 container of ModelIR + RotationSet).
 *
 * Layout (writer src/quant/output.cpp:396-482, reader :484-595): a 54-byte
 * little-endian header {"INTFER1\0", u32 version, u32 n_tensors, u64
 * code_len, u64 scale_len, u64 global_len, u32 n_rotations, u16 reserved,
 * u64 json_len}; json_len bytes of JSON metadata (model_id, n_layers,
 * version, tensors[], rotations[]); the code, scale and global regions; the
 * fp32 rotation matrices (dim x dim, row-major, at each rotation's offset).
 * A quantized tensor's codes are group-major, idx[g*N*G + n*G + (k - g*G)],
 * packed least-significant bits first (dashq.cpp:387-402, :636-672); its
 * scales are one fp16 per K-group shared by all N rows; its global region
 * optionally holds an fp32 alpha.  FP16 tensors hold raw fp16 [N][K].
 * ---------------------------------------------------------------------- */
/* QuantScheme, TensorRole and RotationSite values of include/intfer/quant_spec.h:13-33
 * and include/intfer/spinquant.hpp:45. */
enum { IFR_SCHEME_FP16 = 0, IFR_SCHEME_INT8 = 1, IFR_SCHEME_INT4 = 2, IFR_SCHEME_INT2 = 3 };
enum {
  IFR_ROLE_EMBED = 0, IFR_ROLE_LM_HEAD = 1, IFR_ROLE_ATTN_Q = 2, IFR_ROLE_ATTN_K = 3,
  IFR_ROLE_ATTN_V = 4, IFR_ROLE_ATTN_O = 5, IFR_ROLE_MLP_GATE = 6, IFR_ROLE_MLP_UP = 7,
  IFR_ROLE_MLP_DOWN = 8, IFR_ROLE_NORM = 9, IFR_ROLE_ROPE = 10, IFR_ROLE_OTHER = 17
};
enum { IFR_SITE_QKV = 0, IFR_SITE_O = 1, IFR_SITE_FFN_IN = 2, IFR_SITE_FFN_OUT = 3, IFR_SITE_NONE = 4 };

typedef struct ifr_intfer ifr_intfer;

/* One TensorIR entry (quant_spec.h:48-72) as stored in the file. */
typedef struct ifr_intfer_tensor {
  const char* name;  /* valid while the handle lives */
  int32_t role;      /* IFR_ROLE_* (names outside the table read as OTHER) */
  int32_t N, K;
  int32_t scheme;    /* IFR_SCHEME_* */
  int32_t group_size;
  int32_t scale_dtype;        /* 0 FP16, 1 FP8_E4M3 */
  int32_t has_global_divisor;
  int32_t act;                /* 0 FP16, 1 BF16, 2 INT8_G64 (recorded, not used) */
  int32_t rotation_id;
  uint64_t code_offset, code_bytes, scale_offset, scale_bytes, global_offset, global_bytes;
  float est_error;
} ifr_intfer_tensor;

typedef struct ifr_intfer_rotation {
  int32_t id, site, dim;
  int32_t hadamard; /* 1: exactly the canonical Sylvester H_p / sqrt(p) (with an
                     * identity tail past p = the largest power of two <= dim),
                     * the only rotation the quantizer emits (spinquant.cpp:99-125) */
} ifr_intfer_rotation;

/* Parse a file image (deserialize_intfer_borrowed, output.cpp:484-603).  The
 * handle borrows blob, which must outlive it.  IFR_EINVAL for a malformed or
 * truncated image (the reference's `false`). */
int ifr_intfer_open(const void* blob, size_t n, ifr_intfer** out);
int ifr_intfer_close(ifr_intfer* f);
/* Counts and the JSON's model_id (copied NUL-terminated into buf[0..cap)). */
int ifr_intfer_counts(const ifr_intfer* f, int32_t* n_tensors, int32_t* n_rotations,
                      int32_t* n_layers);
int ifr_intfer_model_id(const ifr_intfer* f, char* buf, size_t cap);
int ifr_intfer_tensor_info(const ifr_intfer* f, int32_t i, ifr_intfer_tensor* out);
/* Index of the tensor named `name` (the last one, if repeated); IFR_EINVAL if absent. */
int ifr_intfer_find(const ifr_intfer* f, const char* name, int32_t* index);
/* Rotation i; mat (may be NULL) receives its dim*dim fp32 matrix. */
int ifr_intfer_rotation_info(const ifr_intfer* f, int32_t i, ifr_intfer_rotation* out, float* mat);
/* Dequantize tensor i to fp32 [N][K] (dequant_tensor, dashq.cpp:696-707,
 * QuantResult::dequant :531-575): w = (fp16(s_g) * alpha) * cb[code] with
 * the canonical codebook cb[c] = (2c - C)/C (INT2 {-1, -1/3, 1/3, 1},
 * :405-417), or the raw fp16 value for an FP16 tensor. */
int ifr_intfer_dequant(const ifr_intfer* f, int32_t i, float* out);

/* Build a host model from the file for the architecture `cfg` (the
 * reference reads it from config.json, main.cpp:10705-10755).  Tensors are
 * found by their Hugging Face names (main.cpp:4225-4270, :10838-10870):
 * model.language_model.{embed_tokens,norm}.weight, [model.language_model.]
 * lm_head.weight (optional, else tied), and per layer L
 * model.language_model.layers.L.{input_layernorm,post_attention_layernorm,
 * self_attn.q_norm,self_attn.k_norm,self_attn.{q,k,v,o}_proj,
 * mlp.{gate,up,down}_proj}.weight.  Linears are mapped exactly (row-major
 * codes, scale(n,g) = s_g, zero = C/2, post = 2*alpha/C, shard_weight
 * engine.cpp:434-549); FP16 or quantized embeddings and norms are
 * dequantized to fp32.  cfg->rotate is set from the file: 1 when every
 * linear's rotation (looked up by rotation_id, main.cpp:839-850) is the
 * canonical Hadamard of the hidden size, 0 when none has one.
 * cfg->attn_gate is set from the file as well: 1 when q_proj has
 * 2 * n_heads * head_dim rows ([q, gate] per head, main.cpp:7624-7640).
 * IFR_EDECLINE for content this engine does not run: FP16 / FP8-scale /
 * non-128-group linears, dense rotations, or a mix of rotated and
 * unrotated linears.  Free the model
 * with ifr_host_model_free; it does not borrow the file. */
int ifr_intfer_host_model(const ifr_intfer* f, const ifr_model_cfg* cfg, ifr_host_model** out);

/* Serialize a host model (serialize_intfer, output.cpp:396-482, byte for
 * byte the reference writer's output for the same ModelIR).  Each linear
 * must have the container's form (one scale per group for all rows, zero =
 * C/2, group 128; else IFR_EDECLINE); alpha = post*C/2 is written as a
 * global divisor unless it is 1.  Embedding, norms and lm_head are written
 * as FP16 tensors.  With cfg.rotate the four shared Hadamard rotations of
 * the hidden size are written (ids 1 + site, spinquant.cpp:505-513).  *out
 * is allocated by the library; release it with ifr_intfer_buffer_free. */
int ifr_intfer_write(const ifr_host_model* m, const char* model_id, void** out, size_t* n);
void ifr_intfer_buffer_free(void* p);

/* ifr_intfer_host_model + ifr_model_load in one call (replaces Engine::load
 * of an .intfer path + ensure_shard_built, engine.cpp:552-743); the file
 * variant maps the file read-only for the duration of the call. */
int ifr_model_load_intfer(ifr_ctx* ctx, const void* blob, size_t n, const ifr_model_cfg* cfg,
                          const ifr_kv_cfg* kv);
int ifr_model_load_intfer_file(ifr_ctx* ctx, const char* path, const ifr_model_cfg* cfg,
                               const ifr_kv_cfg* kv);

/* ------------------------------------------------------------------------
 * Scheduler / serve (C++ host side above the ABI).
 * ---------------------------------------------------------------------- */
typedef struct ifr_sched ifr_sched;

typedef struct ifr_sched_cfg {
  int32_t chunk_m;    /* prefill rows per iteration (INTFER_PREFILL_CHUNK_M, default 128) */
  int32_t live_cap;   /* live decode cap (serve_live_cap, <= 64) */
  int32_t split_iter; /* 1: split path (chunk forward, then decode forward) */
  int32_t round_robin;/* 1: rotate unfilled prefill heads (INTFER_PREFILL_RR) */
  int32_t spec_k;     /* n-gram draft width for verify rows; 0 = off */
  int32_t pack_prefill; /* no reference counterpart (its chunk holds only the
                         * queue head's rows, main.cpp:8447-8470): 1 fills
                         * the chunk_m budget from the prefill queue in
                         * order, so a prompt ending mid-chunk leaves its
                         * room to the next.  Token streams are unchanged. */
  int32_t prefix_cache; /* prefix reuse entries (PrefixCache, main.cpp:
                         * 9469-9726, INTFER_PCACHE_N, at most 16); 0 = off.
                         * A finished request's stream and KV stay cached
                         * (LRU); an admitted prompt sharing a prefix with a
                         * cached stream copies that KV and prefills only the
                         * rest.  Token streams are unchanged. */
  uint32_t seed;        /* base seed of the requests' samplers: a request
                         * without its own seed draws from mt19937(seed + id)
                         * (run_serve admission, main.cpp:9305) */
  int32_t spec_adapt;   /* adaptive draft width (SpecAdapt, main.cpp:
                         * 11454-11511, INTFER_SPEC_ADAPT): 1 picks each
                         * round's width per request as the w in 1..cap
                         * maximising w * accept_ema / (w + 1), with
                         * accept_ema an EMA (0.75 / 0.25, clamped to
                         * [0.05, 0.95], start 0.5) of accepted / drafted;
                         * cap = spec_k, or 8 when spec_k is 0 */
} ifr_sched_cfg;

int ifr_sched_create(ifr_ctx* ctx, const ifr_sched_cfg* cfg, ifr_sched** out);

/* The scheduler talks to its model through this table, the counterpart of
 * the reference scheduler calling step_batch over a LinearBackend
 * (main.cpp:455-566).  ifr_sched_create fills it with the engine's own
 * entry points; a test may pass another model (e.g. a CPU checker). */
typedef struct ifr_sched_backend {
  void* user;
  int (*seq_open)(void* user, int32_t* slot);
  int (*seq_close)(void* user, int32_t slot);
  int (*seq_truncate)(void* user, int32_t slot, int32_t len);
  int (*forward)(void* user, const ifr_row* rows, int32_t M, int32_t* best);
  int32_t kv_capacity;
  /* ifr_seq_copy_prefix; may be NULL (no prefix cache) */
  int (*seq_copy_prefix)(void* user, int32_t dst, int32_t src, int32_t len);
  /* the forward that also returns the logits of the rows with want = 2
   * (ifr_forward's logits_out), [n][vocab] in row order; may be NULL (then
   * only greedy requests are accepted) */
  int (*forward_logits)(void* user, const ifr_row* rows, int32_t M, int32_t* best, float* logits);
  int32_t vocab;
} ifr_sched_backend;
int ifr_sched_create_backend(const ifr_sched_backend* be, const ifr_sched_cfg* cfg,
                             ifr_sched** out);
int ifr_sched_destroy(ifr_sched* s);
/* Admit a request (prompt token ids, max_new).  Returns its id. */
int ifr_sched_submit(ifr_sched* s, const int32_t* prompt, int32_t n, int32_t max_new,
                     int64_t* id);

/* Per-request sampling (Request::temperature / top_k / top_p / rng,
 * main.cpp:4812-4815).  A request is greedy when temperature <= 0, top_k
 * == 0 and top_p <= 0 (main.cpp:8401, :8505): its decode tokens are the
 * device argmax.  Otherwise each decode row's token is ifr_sample over the
 * row's logits with the request's own mt19937, seeded with `seed` when
 * has_seed, else with the scheduler's seed + the request id
 * (main.cpp:9305).  The token that completes a prompt is the argmax in
 * either case (main.cpp:8522-8523, :8366), and a sampling request gets no
 * n-gram verify rows (their acceptance is greedy, main.cpp:11869-11883). */
typedef struct ifr_sample_params {
  float temperature;
  int32_t top_k;
  float top_p;
  uint32_t seed;
  int32_t has_seed;
} ifr_sample_params;
/* ifr_sched_submit with sampling parameters (NULL: greedy).  IFR_EDECLINE
 * for a sampling request when the backend has no forward_logits. */
int ifr_sched_submit_sampled(ifr_sched* s, const int32_t* prompt, int32_t n, int32_t max_new,
                             const ifr_sample_params* sp, int64_t* id);

/* The sampler itself (sample, main.cpp:8674-8764), for one row of logits:
 * temperature <= 0 is read as 1e-5; p = softmax((l - max) / T) with a
 * sequential sum; top_k > 0 keeps the p >= the k-th largest and
 * renormalises; 0 < top_p < 1 keeps the shortest most-probable prefix
 * whose sum reaches top_p and renormalises; the token is the first whose
 * running sum reaches r = U[0,1) (std::uniform_real_distribution<float> of
 * the mt19937: float(x) * 2^-32 below 1), else the last.  ifr_rng is the
 * request's std::mt19937 (the C++ standard's engine, seeded with `seed`). */
typedef struct ifr_rng ifr_rng;
int ifr_rng_create(uint32_t seed, ifr_rng** out);
void ifr_rng_free(ifr_rng* r);
/* The next U[0,1) draw of the generator (the sampler's r). */
int ifr_rng_uniform(ifr_rng* r, float* u);
int ifr_sample(const float* logits, int32_t vocab, int32_t top_k, float top_p, float temperature,
               ifr_rng* rng, int32_t* token);
/* Run one serve iteration (serve_iteration, main.cpp:9203-9259).  Returns
 * the number of rows in the forward(s) it ran, 0 when idle. */
int ifr_sched_step(ifr_sched* s, int32_t* rows_run);
/* Generated tokens of a request so far; *done=1 once finished. */
int ifr_sched_result(ifr_sched* s, int64_t id, int32_t* out, int32_t cap, int32_t* n,
                     int32_t* done);
/* Row list of the last forward the scheduler ran (for replay parity). */
int ifr_sched_last_rows(ifr_sched* s, ifr_row* out, int32_t cap, int32_t* n);

/* Streamed output of the scheduler, the events the reference's serve loop
 * prints (run_serve, main.cpp:9285-9291, :9349-9363): one per generated
 * token of a decode or verify row, in row order (the token that completes
 * a prefill is not streamed), then one done event per request that
 * finished in the step, in live order. */
typedef struct ifr_sched_event {
  int64_t id;        /* request id */
  int32_t token;     /* the token, or -1 for a done event */
  int32_t done;      /* 1: the request finished */
  int32_t generated; /* tokens generated so far (done: the final count) */
  int32_t reserved;
} ifr_sched_event;
/* Start (on = 1) or stop recording events; stopping drops undrained ones. */
int ifr_sched_record_events(ifr_sched* s, int32_t on);
/* Move up to cap recorded events, oldest first, into out; *n = how many. */
int ifr_sched_events(ifr_sched* s, ifr_sched_event* out, int32_t cap, int32_t* n);
/* Forget a finished request (IFR_ESTATE while it still runs). */
int ifr_sched_release(ifr_sched* s, int64_t id);
/* Queue sizes and the per-sequence KV capacity in tokens. */
int ifr_sched_info(ifr_sched* s, int32_t* live, int32_t* prefill, int32_t* pending,
                   int32_t* kv_capacity);

/* The --serve JSON-lines loop (run_serve, main.cpp:9260-9377), over file
 * descriptors.  Each input line is one request,
 *   {"prompt_ids":[t0,t1,...], "max_new":N, "id":K,
 *    "temperature":T, "top_k":K, "top_p":P, "seed":S}
 * (max_new defaults to cfg->default_max_new and is clamped to [1, 4096]; a
 * missing id takes the next free one, main.cpp:9329-9342; the sampling keys
 * default to cfg's, top_k is clamped to >= 0 and top_p to [0, 1], and a
 * seed makes the request's sampler independent of its id,
 * parse_serve_line main.cpp:8646-8668).  Token ids stand in for the
 * reference's "prompt" text: this build has no tokenizer, so a line with
 * only "prompt" is answered with an error.  Output lines, flushed per
 * iteration: {"id":K,"token":T} per streamed token, {"id":K,"done":true,
 * "generated":n} when a request finishes, {"error":"..."} (with "id" when
 * known) for a line that is refused.  Input is polled between iterations
 * and read blocking only while nothing runs; the call returns IFR_OK after
 * end of input once every admitted request has finished, or the first
 * forward error. */
typedef struct ifr_serve_cfg {
  int32_t default_max_new; /* 0: 64 (ServeOpts, main.cpp:8563-8568) */
  int32_t vocab;           /* token ids must be below it (0: checked by the forward) */
  /* defaults of the sampling keys (the CLI's -t / -k / -T, main.cpp:10555-10557) */
  float temperature;
  int32_t top_k;
  float top_p;
  uint32_t seed;           /* a line without "seed" samples from mt19937(seed + its id) (-S) */
} ifr_serve_cfg;
int ifr_serve(ifr_sched* s, int32_t in_fd, int32_t out_fd, const ifr_serve_cfg* cfg);

#ifdef __cplusplus
}
#endif
#endif /* INTFER_AMD_H */
