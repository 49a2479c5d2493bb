// Engine: the C-ABI of include/intfer_amd.h over HIP on one gfx950 GPU.
//
// Replaces the reference's Engine + GpuBackend + step_batch device traffic
// (include/intfer/engine.hpp:37-562, examples/intfer_cli/main.cpp:1027-2866,
// :7519-8320): weights, KV and every intermediate stay resident in HBM; one
// ifr_forward enqueues the whole 28-layer mixed iteration on one stream and
// reads back only the argmax ids (and logits when asked).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ifr_half.h"
#include "host_model.h"
#include "ifr_kernels.h"
#include "intfer_amd.h"

using ifrk::DLin;

namespace ifrh {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace ifrh

namespace {

using ifrh::fail;

#define HIPCHK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(e_ == hipErrorInvalidValue ? IFR_EINVAL : IFR_EDEVICE, "%s: %s (%s:%d)", \
                  #expr, hipGetErrorString(e_), __FILE__, __LINE__);                   \
  } while (0)

constexpr int kPage = 32;

constexpr int kSplit = 256;  // default KV tokens per attention unit
constexpr int kAttnTiles = 1;  // 16-column MFMA tiles per attention unit (q-block = 16 / G tokens)

// ---- the no-allocation attention entry point's scratch (ifr_attention_noalloc)
// Limits of one call: rows, attention units (one per (q-block, kv head,
// 256-token KV split)) and the attention row width n_heads * head_dim.
constexpr int kNaRows = 512;
constexpr int kNaUnits = 4096;
constexpr int kNaRowWidth = 8192;
constexpr size_t na_align(size_t x) { return (x + 255) & ~(size_t)255; }
// byte offsets of each region inside the array
constexpr size_t kNaRowsOff = 0;                                                    // ifr_row[kNaRows]
constexpr size_t kNaMapsOff = na_align(kNaRowsOff + (size_t)kNaRows * 5 * 4);      // 9 int32 maps
constexpr size_t kNaMapLen = na_align((size_t)(kNaRows + 1) * 4);
constexpr size_t kNaUnitsOff = kNaMapsOff + 9 * kNaMapLen;                          // AttnUnit[kNaUnits]
constexpr size_t kNaOrderOff = na_align(kNaUnitsOff + (size_t)kNaUnits * 32);      // int32[4 * kNaUnits]
constexpr size_t kNaPartOOff = na_align(kNaOrderOff + (size_t)kNaUnits * 4 * 4);   // fp32 partial O
constexpr size_t kNaPartMLOff = na_align(kNaPartOOff + (size_t)kNaUnits * 16 * kAttnTiles * 128 * 4);
constexpr size_t kNaAqOff = na_align(kNaPartMLOff + (size_t)kNaUnits * 16 * kAttnTiles * 2 * 4);
constexpr size_t kNaAsOff = na_align(kNaAqOff + (size_t)kNaRows * kNaRowWidth);    // combine's int8 codes
constexpr size_t kNaGsOff = na_align(kNaAsOff + (size_t)kNaRows * 4);
constexpr size_t kNaScratchBytes = na_align(kNaGsOff + (size_t)kNaRows * (kNaRowWidth / 128) * 4);

struct Layer {
  DLin qkv[3];     // fused QKV in qkv[0] when all widths match (nqkv = 1)
  int nqkv = 1;
  int qkv_off[3] = {0, 0, 0};
  DLin o, down;
  DLin gu[2];      // paired gate/up in gu[0] (ngu = 1) or separate gate, up
  int ngu = 1;
  float *in_ln = nullptr, *post_ln = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct Timer {
  std::string name;
  hipEvent_t a, b;
  double bytes, flops;
};

struct Stat {
  double ms = 0, bytes = 0, flops = 0;
  int64_t n = 0;
};

struct Seq {
  bool open = false;
  int len = 0;
  std::vector<int> pages;
};

// One lane of the forward: a HIP stream and the workspaces of the
// sub-batch it runs.  ifr_forward may cut a batch into two contiguous
// sub-batches and run them on the two lanes concurrently (the kernels are
// row-independent, so every row's result is the same either way).
struct Lane {
  hipStream_t st = nullptr;
  int32_t* rows_d = nullptr;
  int32_t* rows_h = nullptr;  // pinned
  float* resid = nullptr;
  int8_t* aq = nullptr;
  float* as = nullptr;
  float* gs = nullptr;
  uint16_t* qkv = nullptr;
  uint16_t* qbuf = nullptr;
  uint16_t* gate = nullptr;   // [M][n_heads * head_dim] attention output gate (gated models)
  uint16_t* y = nullptr;
  uint16_t* mg = nullptr;
  uint16_t* gu = nullptr;
  ifrk::PackOut pk{};
  int32_t* row_tok = nullptr;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  int8_t* lm_aq = nullptr;
  float* lm_as = nullptr;
  float* lm_pv = nullptr;
  int32_t* lm_pi = nullptr;
  int32_t* best_d = nullptr;
  int32_t* best_h = nullptr;  // pinned
  float* logits_d = nullptr;  // grown on demand, freed by release_model
  size_t logits_cap = 0;
};

}  // namespace

// Device memory of ifr_attention_noalloc: one copy per GPU, held until the
// process ends.  Host code uses the address hipGetSymbolAddress gives for the
// current device (ifr_ctx::scratch), never this name.
static __device__ __align__(256) uint8_t scratch[kNaScratchBytes];
// Calls of ifr_attention_noalloc on one GPU share that GPU's array; each call
// holds its device's lock from its first launch until its results are back,
// so calls from different threads or contexts run one after the other.
constexpr int kNaLockDevices = 64;
std::mutex g_na_lock[kNaLockDevices];

struct ifr_dlinear {
  DLin d;
};

struct ifr_ctx {
  int device = 0;
  hipStream_t st = nullptr;
  // model
  bool loaded = false;
  ifr_model_cfg cfg{};
  ifr_kv_cfg kv{};
  std::vector<Layer> layers;
  std::vector<void*> allocs;
  float* embed = nullptr;
  float* final_norm = nullptr;
  uint32_t* lm_w = nullptr;
  uint16_t* lm_s = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  // paged KV
  int n_pages = 0, max_pages = 0;
  std::vector<void*> kpool, vpool;
  std::vector<uint16_t*> kscale, vscale;
  int32_t* bt_d = nullptr;
  void** pools_d = nullptr;        // every KV pool (K, V [, scales] per layer), for page copies
  int npools = 0;
  int32_t* copy_idx_d = nullptr;   // [2][max_pages] source / destination pages
  int32_t* bt_h = nullptr;  // pinned
  std::vector<int> free_pages;
  std::vector<Seq> seqs;
  // workspaces: two lanes (stream + buffers of one sub-batch each)
  int maxM = 0, max_units = 0, last_slots = 0;
  Lane lane[2];
  hipEvent_t ev_bt = nullptr;  // block-table uploads done (lane 0 -> lane 1)
  int last_lanes = 0;          // sub-batches of the last forward
  // timing
  bool timing = false;
  hipEvent_t tev[2] = {nullptr, nullptr};  // ifr_timer_begin / _end
  std::vector<Timer> timers;
  std::vector<std::pair<std::string, Stat>> stats;
  // last forward's split (for tests / bench notes)
  int last_split = 0, last_units = 0;
  int qb = 8;  // q-block tokens per attention unit: 16 MFMA columns / GQA group
  uint8_t* scratch = nullptr;  // this device's copy of `scratch` (resolved at ifr_ctx_create)
  // per-linear seam workspaces (ifr_linear_batch & co.), allocated at first
  // use for max_rows rows and freed with the model
  float* sx = nullptr;        // fp32 [maxM][Kmax] input rows
  int8_t* saq = nullptr;      // A tiles
  float* sas = nullptr;       // [maxM] row scales
  float* sgs = nullptr;       // [maxM][Kmax / 128] group code sums
  uint16_t* sy = nullptr;     // fp16 [maxM][Nmax] output
  uint16_t* smg = nullptr;    // fp16 [maxM][inter] SwiGLU output (ifr_mlp_fused)
  std::vector<uint16_t> hy;   // host copy of one chunk's fp16 output

  void* dalloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes == 0 ? 16 : bytes) != hipSuccess) return nullptr;
    allocs.push_back(p);
    return p;
  }
};

namespace {

Stat& stat_of(ifr_ctx* c, const std::string& n) {
  for (auto& s : c->stats)
    if (s.first == n) return s.second;
  c->stats.push_back({n, Stat()});
  return c->stats.back().second;
}

// Bracket one launch with events when timing is on.
struct Scope {
  ifr_ctx* c;
  hipStream_t st;
  Timer t;
  bool on;
  // bytes / flops: the launch's algorithmic HBM bytes and arithmetic work
  Scope(ifr_ctx* c_, hipStream_t st_, const char* name, double bytes, double flops = 0)
      : c(c_), st(st_), on(c_->timing) {
    if (!on) return;
    t.name = name;
    t.bytes = bytes;
    t.flops = flops;
    hipEventCreate(&t.a);
    hipEventCreate(&t.b);
    hipEventRecord(t.a, st);
  }
  ~Scope() {
    if (!on) return;
    hipEventRecord(t.b, st);
    c->timers.push_back(t);
  }
  // nothing was launched: drop the interval
  void cancel() {
    if (!on) return;
    hipEventDestroy(t.a);
    hipEventDestroy(t.b);
    on = false;
  }
};

void add_host_time(ifr_ctx* c, const char* name, double ms) {
  Stat& s = stat_of(c, name);
  s.ms += ms;
  s.n += 1;
}

void flush_timers(ifr_ctx* c) {
  for (auto& t : c->timers) {
    float ms = 0;
    hipEventSynchronize(t.b);
    hipEventElapsedTime(&ms, t.a, t.b);
    Stat& s = stat_of(c, t.name);
    s.ms += ms;
    s.n += 1;
    s.bytes += t.bytes;
    s.flops += t.flops;
    hipEventDestroy(t.a);
    hipEventDestroy(t.b);
  }
  c->timers.clear();
}

int check_linear(const ifr_linear* w) {
  if (!w || !w->codes || !w->scale || !w->zero)
    return fail(IFR_EINVAL, "linear: null buffer");
  if (w->bits != 2 && w->bits != 4 && w->bits != 8)
    return fail(IFR_EDECLINE, "linear: bits %d not in {2,4,8}", w->bits);
  if (w->group != 128) return fail(IFR_EDECLINE, "linear: group %d != 128", w->group);
  if (w->N <= 0 || w->K <= 0 || w->N % 16 || w->K % 128)
    return fail(IFR_EDECLINE, "linear: N %d must be a multiple of 16, K %d of 128", w->N, w->K);
  if (!std::isfinite(w->post)) return fail(IFR_EINVAL, "linear: post not finite");
  return IFR_OK;
}

float post_of(const ifr_linear& w) { return w.post == 0.0f ? 1.0f : w.post; }

size_t code_bytes(int N, int K, int bits) { return (size_t)N * K * bits / 8; }
size_t sz_bytes(int N, int K) { return (size_t)N * (K / 128) * 4; }

// Upload `count` linears with equal bits and K as one device linear.
// pair=1: exactly two (gate, up) interleaved per 16-column tile.
int upload_group(ifr_ctx* c, const ifr_linear* const* ws, int count, int pair, DLin& d,
                 bool own_tracked) {
  const int K = ws[0]->K, bits = ws[0]->bits;
  int N = 0;
  for (int i = 0; i < count; ++i) {
    if (int r = check_linear(ws[i])) return r;
    if (ws[i]->K != K || ws[i]->bits != bits) return fail(IFR_EINVAL, "group: K/bits mismatch");
    if (post_of(*ws[i]) != post_of(*ws[0])) return fail(IFR_EINVAL, "group: post mismatch");
    N += ws[i]->N;
  }
  if (pair && (count != 2 || ws[0]->N != ws[1]->N)) return fail(IFR_EINVAL, "pair: shape mismatch");
  d.N = N;
  d.K = K;
  d.bits = bits;
  d.ng = K / 128;
  d.nsteps = K / 64;
  d.pair = pair;
  d.post = post_of(*ws[0]);
  // codebook zeros (C/2 everywhere, C = 2^bits - 1: 1.5, 7.5 or 127.5 in
  // fp16): the reference's canonical codebook.  INT2 / INT4 ones take the
  // GEMM's two-operation fold, which gives the same bits.
  const uint16_t zc = bits == 2 ? 0x3E00 : bits == 4 ? 0x4780 : 0x57F8;
  d.cb = 1;
  for (int i = 0; i < count && d.cb; ++i)
    for (size_t e = 0; e < (size_t)ws[i]->N * (K / 128); ++e)
      if (ws[i]->zero[e] != zc) { d.cb = 0; break; }
  d.ff = d.cb && bits != 8;
  const size_t cb = code_bytes(N, K, bits), sb = sz_bytes(N, K);
  std::vector<uint32_t> hc(cb / 4), hs(sb / 4);
  int tile_off = 0;
  for (int i = 0; i < count; ++i) {
    if (pair)
      ifrk::pack_linear_host(ws[i]->codes, ws[i]->scale, ws[i]->zero, ws[i]->N, K, bits, hc.data(),
                             hs.data(), 2, i, 0x80u);
    else
      ifrk::pack_linear_host(ws[i]->codes, ws[i]->scale, ws[i]->zero, ws[i]->N, K, bits, hc.data(),
                             hs.data(), 1, tile_off, 0x80u);
    tile_off += ws[i]->N / 16;
  }
  void* pc = nullptr;
  void* ps = nullptr;
  if (own_tracked) {
    pc = c->dalloc(cb);
    ps = c->dalloc(sb);
    if (!pc || !ps) return fail(IFR_ENOMEM, "hipMalloc weights (%zu B)", cb + sb);
  } else {
    HIPCHK(hipMalloc(&pc, cb));
    if (hipMalloc(&ps, sb) != hipSuccess) {
      hipFree(pc);
      return fail(IFR_ENOMEM, "hipMalloc scales");
    }
  }
  HIPCHK(hipMemcpy(pc, hc.data(), cb, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(ps, hs.data(), sb, hipMemcpyHostToDevice));
  d.codes = static_cast<uint32_t*>(pc);
  d.sz = static_cast<uint32_t*>(ps);
  d.bytes = cb + sb;
  return IFR_OK;
}

template <typename T>
int upload(ifr_ctx* c, T** dst, const T* src, size_t n) {
  *dst = static_cast<T*>(c->dalloc(n * sizeof(T)));
  if (!*dst) return fail(IFR_ENOMEM, "hipMalloc %zu B", n * sizeof(T));
  HIPCHK(hipMemcpy(*dst, src, n * sizeof(T), hipMemcpyHostToDevice));
  return IFR_OK;
}

template <typename T>
int walloc(ifr_ctx* c, T** dst, size_t n) {
  *dst = static_cast<T*>(c->dalloc(n * sizeof(T)));
  if (!*dst) return fail(IFR_ENOMEM, "hipMalloc %zu B", n * sizeof(T));
  return IFR_OK;
}

void release_model(ifr_ctx* c) {
  if (c->st) hipStreamSynchronize(c->st);
  for (void* p : c->allocs) hipFree(p);
  c->allocs.clear();
  if (c->lane[1].st) hipStreamSynchronize(c->lane[1].st);
  if (c->bt_h) hipHostFree(c->bt_h);
  c->bt_h = nullptr;
  for (Lane& L : c->lane) {
    for (int32_t** hp : {&L.rows_h, &L.best_h})
      if (*hp) hipHostFree(*hp);
    if (L.logits_d) hipFree(L.logits_d);
    hipStream_t st = L.st;
    L = Lane();
    L.st = st;
  }
  c->layers.clear();
  c->sx = nullptr;
  c->saq = nullptr;
  c->sas = c->sgs = nullptr;
  c->sy = c->smg = nullptr;
  c->kpool.clear();
  c->vpool.clear();
  c->kscale.clear();
  c->vscale.clear();
  c->seqs.clear();
  c->free_pages.clear();
  c->loaded = false;
}

// Units the pack kernel will emit for a given split (same formula).
long count_units(const std::vector<int>& g_pos0, const std::vector<int>& g_len, int nkv, int split,
                 int qb) {
  long n = 0;
  for (size_t g = 0; g < g_len.size(); ++g) {
    const int nb = (g_len[g] + qb - 1) / qb;
    for (int b = 0; b < nb; ++b) {
      const int kvhi = g_pos0[g] + std::min((b + 1) * qb, g_len[g]);
      n += (long)nkv * ((kvhi + split - 1) / split);
    }
  }
  return n;
}

// Attention units the workspace is sized for: the most any admissible batch
// can need.  M <= max_rows rows in at most min(M, max_seqs) sequence groups
// make at most ceil(M / qb) + min(M, max_seqs) q-blocks (each group adds one
// partial block), and a q-block's keys end at most at max_seq_tokens, so it
// has at most ceil(max_seq_tokens / split) splits per kv head.  Capped at
// kMaxUnits (partials of 8 KB each: about 4.4 GB); a capped engine declines
// the batches beyond it.
constexpr long kMaxUnits = 1L << 19;
int max_units_for(const ifr_kv_cfg& kv, int nkv, int qb) {
  const long split = kv.attn_split > 0 ? kv.attn_split : kSplit;
  const long M = kv.max_rows;
  const long qblocks = (M + qb - 1) / qb + std::min<long>(M, kv.max_seqs);
  const long bound = (long)nkv * qblocks * ((kv.max_seq_tokens + split - 1) / split);
  return (int)std::min(bound, kMaxUnits);
}

// Algorithmic work of one attention launch: K+V of every row's sequence
// (plus int8 scales), Q in and O out; flops = QK^T + PV over each row's
// visible keys (pos + 1).
void attn_work(const ifr_ctx* c, const ifr_row* rows, int M, const std::vector<int>& g_pos0,
               const std::vector<int>& g_len, double* bytes, double* flops) {
  const int kvN = c->cfg.n_kv * c->cfg.head_dim, qN = c->cfg.n_heads * c->cfg.head_dim;
  const double e = c->kv.kv_int8 ? 1.0 : 2.0;
  double b = 0, f = 0;
  for (size_t g = 0; g < g_len.size(); ++g) {
    const double Ls = g_pos0[g] + g_len[g];
    b += Ls * kvN * 2 * e + (c->kv.kv_int8 ? Ls * c->cfg.n_kv * 2 * 2 : 0);
  }
  b += (double)M * qN * 2 * 2;
  for (int m = 0; m < M; ++m) f += 4.0 * qN * (rows[m].pos + 1);
  *bytes = b;
  *flops = f;
}

// Bytes the combine pass moves: each row's fp32 partial (O, m, l) of every
// q head over its splits (a q-block's split count is ceil(kv_hi / split)),
// and the int8 row, its scale and group sums out.
double combine_work(const ifr_ctx* c, int M, const std::vector<int>& g_pos0, const std::vector<int>& g_len,
                    int split, int qb) {
  const int nq = c->cfg.n_heads, hd = c->cfg.head_dim;
  double b = (double)M * (nq * hd + 4 + nq * hd / 128 * 4);
  for (size_t g = 0; g < g_len.size(); ++g)
    for (int t = 0; t < g_len[g]; ++t) {
      const int kvhi = g_pos0[g] + std::min((t / qb + 1) * qb, g_len[g]);
      b += (double)nq * ((kvhi + split - 1) / split) * (hd * 4 + 8);
    }
  return b;
}

// Slots of the chunked region whose workgroups share K/V pages through LDS
// (the q-blocks of prefill chunks; fp16 KV); otherwise every slot runs as an
// independent unit, with the same results.
int shared_slots(const ifr_ctx* c, long nchunked) {
  return c->kv.kv_int8 || c->kv.dense_attention ? 0 : (int)nchunked;
}

// Bytes the pack pass moves: the rows in, the per-row maps, the group
// offsets, the units and the dispatch order out.
double pack_work(int M, size_t ngroups, long nunits, int nslots) {
  return (double)M * (5 + 7) * 4 + (double)(ngroups + 1) * 4 + (double)nunits * sizeof(ifrk::AttnUnit) +
         (double)nslots * 4;
}

// Groups of at least this many rows are prefill chunks: ifr_forward runs them
// on lane 1 while the decode / verify rows run on lane 0.
constexpr int kChunkRows = 32;
// Decode-only batches of at least this many rows are halved across the lanes.
constexpr int kMinSplitRows = 16;

// One contiguous sub-batch of an ifr_forward call, run on one lane.
struct SubBatch {
  int lane = 0;
  int row0 = 0, M = 0;             // rows [row0, row0 + M) of the call
  std::vector<int> g_pos0, g_len;  // its sequence groups
  std::vector<int> want;           // scored rows (local indices, ascending)
  std::vector<int> want_logits;    // positions in `want` of the rows with want = 2
  int split = 0, nslots = 0;
  long nunits = 0, nchunked = 0;
  double attn_bytes = 0, attn_flops = 0, comb_bytes = 0, pack_bytes = 0;
};

int prep_sub(ifr_ctx* c, const ifr_row* rows, SubBatch& sb) {
  const ifr_row* r = rows + sb.row0;
  for (int m = 0; m < sb.M; ++m)
    if (r[m].want) {
      if (r[m].want == 2) sb.want_logits.push_back((int)sb.want.size());
      sb.want.push_back(m);
    }
  const int nkv = c->cfg.n_kv;
  // fixed KV split: each row's partial decomposition depends only on its own
  // sequence (batch-invariant results: split == joint, solo == loaded).  The
  // unit workspace is sized at load for the largest batch the engine admits,
  // so only an engine whose bound was capped can see more units; such a
  // batch is declined (nothing enqueued) rather than run with a wider split,
  // which would change every row's decomposition.
  sb.split = c->kv.attn_split > 0 ? c->kv.attn_split : kSplit;
  sb.nunits = count_units(sb.g_pos0, sb.g_len, nkv, sb.split, c->qb);
  if (sb.nunits > c->max_units)
    return fail(IFR_EDECLINE, "batch needs %ld attention units, the workspace holds %d (KV split %d)",
                sb.nunits, c->max_units, sb.split);
  sb.nslots = (int)ifrk::attn_slot_count(sb.g_pos0.data(), sb.g_len.data(), (int)sb.g_len.size(), nkv,
                                         sb.split, c->qb, &sb.nchunked);
  attn_work(c, r, sb.M, sb.g_pos0, sb.g_len, &sb.attn_bytes, &sb.attn_flops);
  sb.comb_bytes = combine_work(c, sb.M, sb.g_pos0, sb.g_len, sb.split, c->qb);
  sb.pack_bytes = pack_work(sb.M, sb.g_len.size(), sb.nunits, sb.nslots);
  if (sb.lane == 0) {
    c->last_split = sb.split;
    c->last_units = (int)sb.nunits;
    c->last_slots = sb.nslots;
  }
  return IFR_OK;
}

// Rows up; the pack kernel writes the packing maps and the token column.
int launch_head(ifr_ctx* c, const ifr_row* rows, const SubBatch& sb) {
  Lane& L = c->lane[sb.lane];
  const ifr_row* r = rows + sb.row0;
  std::memcpy(L.rows_h, r, (size_t)sb.M * sizeof(ifr_row));
  HIPCHK(hipMemcpyAsync(L.rows_d, L.rows_h, (size_t)sb.M * sizeof(ifr_row), hipMemcpyHostToDevice, L.st));
  Scope sc(c, L.st, "pack", sb.pack_bytes);
  HIPCHK(ifrk::launch_pack(L.rows_d, sb.M, c->cfg.n_kv, c->qb, sb.split, L.pk, L.st));
  return IFR_OK;
}

// One decoder layer of a sub-batch on its lane.
int launch_layer(ifr_ctx* c, const SubBatch& sb, int l) {
  const ifr_model_cfg& cf = c->cfg;
  Lane& L = c->lane[sb.lane];
  const int M = sb.M;
  const int H = cf.hidden, hd = cf.head_dim, nq = cf.n_heads, nkv = cf.n_kv;
  const int qN = nq * hd, kvN = nkv * hd, F = cf.inter;
  const int qkvN = (cf.attn_gate ? 2 * qN : qN) + 2 * kvN;  // QKV output width
  Layer& ly = c->layers[l];
  ifrk::KVLayout kv{nkv, hd, kPage, c->max_pages, c->kv.kv_int8, c->kpool[l], c->vpool[l],
                    c->kscale[l], c->vscale[l], c->bt_d};
  // (1) layer input: embed (l == 0) or residual += FWHT(down out); RMSNorm; FWHT; quant
  {
    ifrk::RowQuantArgs a{};
    if (l == 0) {
      a.src = ifrk::SRC_EMBED;
      a.embed = c->embed;
      a.tokens = L.row_tok;
    } else {
      a.src = ifrk::SRC_RESID;
      a.y = L.y;
      a.rot_y = cf.rotate;
    }
    a.resid = L.resid;
    a.norm_w = ly.in_ln;
    a.eps = cf.rms_eps;
    a.rotate = cf.rotate;
    a.round = 0;
    a.ga = 0;
    a.q = L.aq;
    a.qscale = L.as;
    a.gsum = L.gs;
    a.M = M;
    a.K = H;
    Scope sc(c, L.st, "row_quant", (double)M * H * 4 * 2);
    HIPCHK(ifrk::launch_row_quant(a, L.st));
  }
  // (2) QKV and (3) q/k norm + RoPE + KV append: one launch when the QKV
  // GEMM's launch shape holds one head per workgroup, else two passes
  const ifrk::QKArgs qka{L.qkv, L.pk.row_seq, L.pk.row_pos, ly.q_norm, ly.k_norm, c->rope_cos,
                         c->rope_sin, cf.rotary_dim, cf.rms_eps, nq, L.qbuf, M, cf.attn_gate, L.gate};
  bool fused = false;
  if (!c->kv.separate_qk && ly.nqkv == 1) {
    ifrk::QGemmArgs a{L.aq, L.as, L.gs, nullptr, nullptr, M, qkvN};
    Scope sc(c, L.st, "qgemm_qkv", (double)ly.qkv[0].bytes + (double)M * (H + 4) + (double)M * ly.qkv[0].N * 2,
             2.0 * M * ly.qkv[0].N * H);
    const hipError_t e = ifrk::launch_qgemm_qkrope(ly.qkv[0], a, qka, kv, -1, L.st);
    if (e == hipErrorInvalidValue) {
      (void)hipGetLastError();
      sc.cancel();
    } else {
      HIPCHK(e);
      fused = true;
    }
  }
  if (!fused) {
    for (int j = 0; j < ly.nqkv; ++j) {
      ifrk::QGemmArgs a{L.aq, L.as, L.gs, L.qkv + ly.qkv_off[j], nullptr, M, qkvN};
      Scope sc(c, L.st, "qgemm_qkv", (double)ly.qkv[j].bytes + (double)M * (H + 4) + (double)M * ly.qkv[j].N * 2,
               2.0 * M * ly.qkv[j].N * H);
      HIPCHK(ifrk::launch_qgemm(ly.qkv[j], a, L.st));
    }
    Scope sc(c, L.st, "qk_rope_kv", (double)M * qkvN * 2 * 2);
    HIPCHK(ifrk::launch_qk_rope_kv(qka, kv, L.st));
  }
  // (4) attention + combine (emits the O-proj int8 input)
  {
    ifrk::AttnArgs a{L.pk.units, (int)sb.nunits, L.pk.order, sb.nslots, shared_slots(c, sb.nchunked),
                     L.qbuf, nq, 1.4426950408889634f / std::sqrt((float)hd), L.part_o, L.part_ml, kAttnTiles};
    Scope sc(c, L.st, "attention", sb.attn_bytes, sb.attn_flops);
    HIPCHK(ifrk::launch_attention(a, kv, L.st));
  }
  {
    ifrk::CombineArgs a{L.part_o, L.part_ml, L.pk.comb_base, L.pk.comb_nsplit, L.pk.comb_tok,
                        M, nq, nkv, hd, nullptr, L.aq, L.as, L.gs, 16 * kAttnTiles,
                        cf.attn_gate && !cf.attn_gate_off ? L.gate : nullptr};
    Scope sc(c, L.st, "combine", sb.comb_bytes);
    HIPCHK(ifrk::launch_combine(a, L.st));
  }
  // (5) O projection
  {
    ifrk::QGemmArgs a{L.aq, L.as, L.gs, L.y, nullptr, M, H};
    Scope sc(c, L.st, "qgemm_o", (double)ly.o.bytes + (double)M * (qN + 4) + (double)M * H * 2,
             2.0 * M * H * qN);
    HIPCHK(ifrk::launch_qgemm(ly.o, a, L.st));
  }
  // (6) residual += FWHT(o); post norm; FWHT; quant
  {
    ifrk::RowQuantArgs a{};
    a.src = ifrk::SRC_RESID;
    a.y = L.y;
    a.rot_y = cf.rotate;
    a.resid = L.resid;
    a.norm_w = ly.post_ln;
    a.eps = cf.rms_eps;
    a.rotate = cf.rotate;
    a.q = L.aq;
    a.qscale = L.as;
    a.gsum = L.gs;
    a.M = M;
    a.K = H;
    Scope sc(c, L.st, "row_quant", (double)M * H * 4 * 2);
    HIPCHK(ifrk::launch_row_quant(a, L.st));
  }
  // (7) gate/up + SwiGLU
  if (ly.ngu == 1) {
    ifrk::QGemmArgs a{L.aq, L.as, L.gs, L.mg, nullptr, M, F};
    Scope sc(c, L.st, "qgemm_gate_up", (double)ly.gu[0].bytes + (double)M * (H + 4) + (double)M * F * 2,
             2.0 * M * 2 * F * H);
    HIPCHK(ifrk::launch_qgemm(ly.gu[0], a, L.st));
  } else {
    for (int j = 0; j < 2; ++j) {
      ifrk::QGemmArgs a{L.aq, L.as, L.gs, L.gu + j * F, nullptr, M, 2 * F};
      Scope sc(c, L.st, "qgemm_gate_up", (double)ly.gu[j].bytes + (double)M * (H + 4) + (double)M * F * 2,
               2.0 * M * F * H);
      HIPCHK(ifrk::launch_qgemm(ly.gu[j], a, L.st));
    }
    HIPCHK(ifrk::launch_swiglu(L.gu, M, F, L.mg, L.st));
  }
  // (8) quantize mg, down projection
  {
    Scope sc(c, L.st, "quant_plain", (double)M * F * 3);
    HIPCHK(ifrk::launch_quant_plain(nullptr, L.mg, M, F, L.aq, L.as, L.gs, L.st));
  }
  {
    ifrk::QGemmArgs a{L.aq, L.as, L.gs, L.y, nullptr, M, H};
    Scope sc(c, L.st, "qgemm_down", (double)ly.down.bytes + (double)M * (F + 4) + (double)M * H * 2,
             2.0 * M * H * F);
    HIPCHK(ifrk::launch_qgemm(ly.down, a, L.st));
  }
  return IFR_OK;
}

// Final residual, norm, lm_head + argmax on the scored rows; the tokens (and
// logits, into logits_out when given: every scored row's, or with only_2 the
// rows with want = 2) come back on the lane's stream.
int launch_tail(ifr_ctx* c, const SubBatch& sb, float* logits_out, bool only_2) {
  const ifr_model_cfg& cf = c->cfg;
  Lane& L = c->lane[sb.lane];
  const int nwant = (int)sb.want.size();
  if (nwant == 0) return IFR_OK;
  const int H = cf.hidden, V = cf.vocab;
  {
    ifrk::RowQuantArgs a{};
    a.src = ifrk::SRC_RESID;
    a.y = L.y;
    a.rot_y = cf.rotate;
    a.resid = L.resid;
    a.rowmap = L.pk.want_rows;
    a.norm_w = c->final_norm;
    a.eps = cf.rms_eps;
    a.rotate = 0;
    a.round = 1;
    a.ga = 64;
    a.q = L.lm_aq;
    a.qscale = L.lm_as;
    a.gsum = nullptr;
    a.M = nwant;
    a.K = H;
    Scope sc(c, L.st, "row_quant", (double)nwant * H * 4 * 2);
    HIPCHK(ifrk::launch_row_quant(a, L.st));
  }
  if (logits_out && L.logits_cap < (size_t)nwant * V) {
    HIPCHK(hipStreamSynchronize(L.st));
    if (L.logits_d) HIPCHK(hipFree(L.logits_d));
    L.logits_d = nullptr;
    HIPCHK(hipMalloc(reinterpret_cast<void**>(&L.logits_d), (size_t)nwant * V * sizeof(float)));
    L.logits_cap = (size_t)nwant * V;
  }
  ifrk::LmHeadArgs a{};
  a.a = L.lm_aq;
  a.as = L.lm_as;
  a.wcodes = c->lm_w;
  a.wscale = c->lm_s;
  a.W = nwant;
  a.V = V;
  a.H = H;
  a.logits = logits_out ? L.logits_d : nullptr;
  a.part_val = L.lm_pv;
  a.part_idx = L.lm_pi;
  a.best = L.best_d;
  {
    Scope sc(c, L.st, "lmhead", (double)V * H + (double)V * 2 + (double)nwant * H);
    HIPCHK(ifrk::launch_lmhead(a, L.st));
  }
  HIPCHK(hipMemcpyAsync(L.best_h, L.best_d, nwant * sizeof(int32_t), hipMemcpyDeviceToHost, L.st));
  if (logits_out && !only_2)
    HIPCHK(hipMemcpyAsync(logits_out, L.logits_d, (size_t)nwant * V * sizeof(float), hipMemcpyDeviceToHost,
                          L.st));
  if (logits_out && only_2)
    for (size_t j = 0; j < sb.want_logits.size(); ++j)
      HIPCHK(hipMemcpyAsync(logits_out + j * V, L.logits_d + (size_t)sb.want_logits[j] * V, (size_t)V * sizeof(float),
                            hipMemcpyDeviceToHost, L.st));
  return IFR_OK;
}

}  // namespace

extern "C" {

const char* ifr_last_error(void) { return ifrh::g_err.c_str(); }

int ifr_ctx_create(int32_t device, ifr_ctx** out) {
  if (!out) return fail(IFR_EINVAL, "out is null");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(IFR_EDEVICE, "no HIP device");
  if (device < 0 || device >= n) return fail(IFR_EINVAL, "device %d of %d", device, n);
  HIPCHK(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(IFR_EDEVICE, "device %d is %s; this build targets gfx950", device, prop.gcnArchName);
  auto* c = new ifr_ctx();
  c->device = device;
  // two default-priority streams: the primary one (c->st, lane 0) and lane 1
  if (hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(IFR_EDEVICE, "hipStreamCreate");
  }
  if (hipStreamCreateWithFlags(&c->lane[1].st, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&c->ev_bt, hipEventDisableTiming) != hipSuccess) {
    hipStreamDestroy(c->st);
    if (c->lane[1].st) hipStreamDestroy(c->lane[1].st);
    delete c;
    return fail(IFR_EDEVICE, "hipStreamCreate (lane 1)");
  }
  c->lane[0].st = c->st;
  // the device's copy of the no-allocation scratch array, with the device current
  void* sp = nullptr;
  const hipError_t es = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
  if (es != hipSuccess || !sp) {
    hipEventDestroy(c->ev_bt);
    hipStreamDestroy(c->lane[1].st);
    hipStreamDestroy(c->st);
    delete c;
    return fail(IFR_EDEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(es));
  }
  c->scratch = static_cast<uint8_t*>(sp);
  *out = c;
  return IFR_OK;
}

int ifr_ctx_destroy(ifr_ctx* c) {
  if (!c) return IFR_OK;
  hipSetDevice(c->device);
  release_model(c);
  for (hipEvent_t& e : c->tev)
    if (e) hipEventDestroy(e);
  if (c->ev_bt) hipEventDestroy(c->ev_bt);
  if (c->lane[1].st) hipStreamDestroy(c->lane[1].st);
  if (c->st) hipStreamDestroy(c->st);
  delete c;
  return IFR_OK;
}

void* ifr_ctx_stream(ifr_ctx* c) { return c ? (void*)c->st : nullptr; }

int ifr_timer_begin(ifr_ctx* c) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  if (!c->tev[0]) {
    HIPCHK(hipEventCreate(&c->tev[0]));
    HIPCHK(hipEventCreate(&c->tev[1]));
  }
  HIPCHK(hipEventRecord(c->tev[0], c->st));
  return IFR_OK;
}

int ifr_timer_end(ifr_ctx* c, double* ms) {
  if (!c || !ms) return fail(IFR_EINVAL, "null arg");
  if (!c->tev[0]) return fail(IFR_ESTATE, "ifr_timer_begin not called");
  HIPCHK(hipEventRecord(c->tev[1], c->st));
  HIPCHK(hipEventSynchronize(c->tev[1]));
  float f = 0;
  HIPCHK(hipEventElapsedTime(&f, c->tev[0], c->tev[1]));
  *ms = f;
  return IFR_OK;
}

int ifr_sync(ifr_ctx* c) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipStreamSynchronize(c->st));
  return IFR_OK;
}

int ifr_malloc(ifr_ctx* c, size_t bytes, void** p) {
  if (!c || !p) return fail(IFR_EINVAL, "null arg");
  if (hipMalloc(p, bytes == 0 ? 16 : bytes) != hipSuccess) return fail(IFR_ENOMEM, "hipMalloc %zu", bytes);
  return IFR_OK;
}
int ifr_free(ifr_ctx* c, void* p) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipStreamSynchronize(c->st));
  HIPCHK(hipFree(p));
  return IFR_OK;
}
int ifr_h2d(ifr_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return IFR_OK;
}
int ifr_d2h(ifr_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return IFR_OK;
}
int ifr_d2d(ifr_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->st));
  return IFR_OK;
}
int ifr_memset(ifr_ctx* c, void* dst, int v, size_t bytes) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  HIPCHK(hipMemsetAsync(dst, v, bytes, c->st));
  return IFR_OK;
}

// ---- kernel-level entry points ------------------------------------------------

int ifr_linear_upload(ifr_ctx* c, const ifr_linear* w, ifr_dlinear** out) {
  if (!c || !out) return fail(IFR_EINVAL, "null arg");
  auto* d = new ifr_dlinear();
  const ifr_linear* ws[1] = {w};
  if (int r = upload_group(c, ws, 1, 0, d->d, false)) { delete d; return r; }
  *out = d;
  return IFR_OK;
}

int ifr_linear_upload_pair(ifr_ctx* c, const ifr_linear* gate, const ifr_linear* up,
                           ifr_dlinear** out) {
  if (!c || !out) return fail(IFR_EINVAL, "null arg");
  auto* d = new ifr_dlinear();
  const ifr_linear* ws[2] = {gate, up};
  if (int r = upload_group(c, ws, 2, 1, d->d, false)) { delete d; return r; }
  *out = d;
  return IFR_OK;
}

int ifr_linear_free(ifr_ctx* c, ifr_dlinear* w) {
  if (!w) return IFR_OK;
  if (c) hipStreamSynchronize(c->st);
  hipFree(w->d.codes);
  hipFree(w->d.sz);
  delete w;
  return IFR_OK;
}

size_t ifr_linear_bytes(const ifr_dlinear* w) { return w ? w->d.bytes : 0; }

int ifr_act_quant(ifr_ctx* c, const float* x_d, int32_t M, int32_t K, const float* norm_w_d,
                  float eps, int32_t rotate, int32_t round, int32_t ga, int8_t* q_d,
                  float* scale_d, float* gsum_d) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  ifrk::RowQuantArgs a{};
  a.src = ifrk::SRC_X;
  a.x = x_d;
  a.norm_w = norm_w_d;
  a.eps = eps;
  a.rotate = rotate;
  a.round = round;
  a.ga = ga;
  a.q = q_d;
  a.qscale = scale_d;
  a.gsum = gsum_d;
  a.M = M;
  a.K = K;
  HIPCHK(ifrk::launch_row_quant(a, c->st));
  return IFR_OK;
}

int ifr_quant_gemm(ifr_ctx* c, const ifr_dlinear* w, const int8_t* a_d, const float* ascale_d,
                   const float* gsum_d, int32_t M, uint16_t* out_d, int32_t* tdump_d) {
  if (!c || !w) return fail(IFR_EINVAL, "null arg");
  if (w->d.pair) return fail(IFR_EINVAL, "paired linear: use ifr_quant_gemm_swiglu");
  ifrk::QGemmArgs a{a_d, ascale_d, gsum_d, out_d, tdump_d, M, w->d.N};
  HIPCHK(ifrk::launch_qgemm(w->d, a, c->st));
  return IFR_OK;
}

int ifr_quant_gemm_swiglu(ifr_ctx* c, const ifr_dlinear* w, const int8_t* a_d,
                          const float* ascale_d, const float* gsum_d, int32_t M, uint16_t* out_d) {
  if (!c || !w) return fail(IFR_EINVAL, "null arg");
  if (!w->d.pair) return fail(IFR_EINVAL, "linear is not a gate/up pair");
  ifrk::QGemmArgs a{a_d, ascale_d, gsum_d, out_d, nullptr, M, w->d.N / 2};
  HIPCHK(ifrk::launch_qgemm(w->d, a, c->st));
  return IFR_OK;
}

int ifr_quant_gemm_f16(ifr_ctx* c, const ifr_dlinear* w, const uint16_t* a_d, int32_t M, float alpha,
                       uint16_t* out_d) {
  if (!c || !w || !a_d || !out_d) return fail(IFR_EINVAL, "null arg");
  if (w->d.pair) return fail(IFR_EDECLINE, "fp16 GEMM: gate/up pairs are not supported");
  if (!w->d.cb) return fail(IFR_EDECLINE, "fp16 GEMM: needs the canonical codebook (zero = C/2 in every group)");
  if (M <= 0) return fail(IFR_EINVAL, "M=%d", M);
  if (M == 1 && w->d.K > 32768) return fail(IFR_EDECLINE, "fp16 GEMM: K=%d above 32768 at M = 1", w->d.K);
  const ifrk::F16Args p{a_d, w->d.codes, w->d.sz, out_d, M, w->d.N, w->d.K, w->d.bits, w->d.nsteps, w->d.ng, alpha};
  HIPCHK(ifrk::launch_qgemm_f16(p, c->st));
  return IFR_OK;
}

int ifr_quant_gemm_ga(ifr_ctx* c, const ifr_dlinear* w, const int8_t* a_d, const float* ascale_d, int32_t M,
                      int32_t ga, float alpha, uint16_t* out_d) {
  if (!c || !w || !a_d || !ascale_d || !out_d) return fail(IFR_EINVAL, "null arg");
  if (w->d.pair) return fail(IFR_EDECLINE, "grouped-activation GEMM: gate/up pairs are not supported");
  if (!w->d.cb)
    return fail(IFR_EDECLINE, "grouped-activation GEMM: needs the canonical codebook (zero = C/2 in every group)");
  if (M <= 0) return fail(IFR_EINVAL, "M=%d", M);
  if (ga == 0) ga = w->d.K;
  if (ga < 0 || ga % 64 != 0 || w->d.K % ga != 0)
    return fail(IFR_EINVAL, "ga=%d: a multiple of 64 dividing K=%d (0: K)", ga, w->d.K);
  const ifrk::GaArgs p{a_d, ascale_d, w->d.codes, w->d.sz, out_d, M, w->d.N, w->d.K, w->d.bits,
                       w->d.nsteps, w->d.ng, ga, alpha};
  HIPCHK(ifrk::launch_qgemm_ga(p, c->st));
  return IFR_OK;
}

int ifr_quant_gemm_variants(void) { return ifrk::kQGemmVariants; }

int ifr_quant_gemm_rows(ifr_ctx* c, const ifr_dlinear* w, const int8_t* a_d, const int8_t* arow_d,
                        const float* ascale_d, const float* gsum_d, int32_t M, uint16_t* out_d, int32_t variant) {
  if (!c || !w) return fail(IFR_EINVAL, "null arg");
  if (variant < -1 || variant >= ifrk::kQGemmVariants) return fail(IFR_EINVAL, "variant %d", variant);
  ifrk::QGemmArgs a{a_d, ascale_d, gsum_d, out_d, nullptr, M, w->d.pair ? w->d.N / 2 : w->d.N, arow_d};
  const hipError_t e = ifrk::launch_qgemm_variant(w->d, a, variant, c->st);
  if (e == hipErrorInvalidValue && variant >= 0) {
    (void)hipGetLastError();
    return fail(IFR_EDECLINE, "variant %d does not apply to M=%d N=%d K=%d", variant, M, w->d.N, w->d.K);
  }
  HIPCHK(e);
  return IFR_OK;
}

int ifr_quant_gemm_variant(ifr_ctx* c, const ifr_dlinear* w, const int8_t* a_d,
                           const float* ascale_d, const float* gsum_d, int32_t M, uint16_t* out_d,
                           int32_t variant) {
  if (!c || !w) return fail(IFR_EINVAL, "null arg");
  if (variant < 0 || variant >= ifrk::kQGemmVariants) return fail(IFR_EINVAL, "variant %d", variant);
  ifrk::QGemmArgs a{a_d, ascale_d, gsum_d, out_d, nullptr, M, w->d.pair ? w->d.N / 2 : w->d.N};
  const hipError_t e = ifrk::launch_qgemm_variant(w->d, a, variant, c->st);
  if (e == hipErrorInvalidValue) {
    (void)hipGetLastError();
    return fail(IFR_EDECLINE, "variant %d does not apply to M=%d N=%d K=%d", variant, M, w->d.N, w->d.K);
  }
  HIPCHK(e);
  return IFR_OK;
}

// ---- model load ------------------------------------------------------------------

int ifr_model_load(ifr_ctx* c, const ifr_host_model* m, const ifr_kv_cfg* kvc) {
  if (!c || !m || !kvc) return fail(IFR_EINVAL, "null arg");
  HIPCHK(hipSetDevice(c->device));
  const ifr_model_cfg& cf = m->cfg;
  if (cf.layers <= 0 || cf.n_heads <= 0 || cf.n_kv <= 0 || cf.vocab <= 0 || cf.hidden <= 0 || cf.inter <= 0 ||
      !m->layers || !m->embed || !m->final_norm)
    return fail(IFR_EINVAL, "model cfg / buffers");
  if (cf.head_dim != 128) return fail(IFR_EDECLINE, "head_dim %d != 128", cf.head_dim);
  // every per-kernel shape limit is checked here, so no forward can fail
  // part-way through a layer because of the model's shape: the attention
  // combine holds one row of n_heads * head_dim <= 8192 in a workgroup
  if (cf.n_heads * cf.head_dim > 8192)
    return fail(IFR_EDECLINE, "n_heads * head_dim = %d > 8192", cf.n_heads * cf.head_dim);
  if (cf.n_heads % cf.n_kv != 0 || cf.n_heads / cf.n_kv > 8)
    return fail(IFR_EDECLINE, "GQA group %d/%d unsupported", cf.n_heads, cf.n_kv);
  if (cf.hidden % 256 || cf.hidden > 8192 || (cf.n_heads * cf.head_dim) % 256 ||
      cf.inter % 128 || cf.inter > ifrk::kQuantPlainMaxK || cf.vocab % 16)
    return fail(IFR_EDECLINE, "model shape unsupported");
  if (cf.rotary_dim <= 0 || cf.rotary_dim > cf.head_dim || cf.rotary_dim % 2)
    return fail(IFR_EINVAL, "rotary_dim");
  if (kvc->max_seqs <= 0 || kvc->max_seq_tokens <= 0 || kvc->pool_tokens < kPage ||
      kvc->max_rows <= 0 || kvc->max_rows > 6144 || kvc->attn_split < 0 || kvc->attn_split % kPage ||
      kvc->attn_split > 65536 || kvc->lanes < 0 || kvc->lanes > 2 || kvc->dense_attention < 0 ||
      kvc->dense_attention > 1)
    return fail(IFR_EINVAL, "kv cfg");
  release_model(c);
  c->cfg = cf;
  c->kv = *kvc;
  c->qb = 16 * kAttnTiles / (cf.n_heads / cf.n_kv);
  const int H = cf.hidden, L = cf.layers, hd = cf.head_dim, nq = cf.n_heads, nkv = cf.n_kv;
  const int qN = nq * hd, kvN = nkv * hd, F = cf.inter, V = cf.vocab;
  c->layers.resize(L);
  for (int l = 0; l < L; ++l) {
    const ifr_layer_w& lw = m->layers[l];
    Layer& ly = c->layers[l];
    if (lw.q.N != (cf.attn_gate ? 2 * qN : qN) || lw.k.N != kvN || lw.v.N != kvN || lw.o.N != H || lw.o.K != qN ||
        lw.gate.N != F || lw.up.N != F || lw.down.N != H || lw.down.K != F || lw.q.K != H)
      return fail(IFR_EINVAL, "layer %d: linear shapes do not match the config", l);
    if (lw.q.bits == lw.k.bits && lw.q.bits == lw.v.bits && post_of(lw.q) == post_of(lw.k) &&
        post_of(lw.q) == post_of(lw.v)) {
      const ifr_linear* ws[3] = {&lw.q, &lw.k, &lw.v};
      ly.nqkv = 1;
      if (int r = upload_group(c, ws, 3, 0, ly.qkv[0], true)) return r;
    } else {
      ly.nqkv = 3;
      const ifr_linear* ws[3] = {&lw.q, &lw.k, &lw.v};
      int off = 0;
      for (int j = 0; j < 3; ++j) {
        if (int r = upload_group(c, &ws[j], 1, 0, ly.qkv[j], true)) return r;
        ly.qkv_off[j] = off;
        off += ws[j]->N;
      }
    }
    {
      const ifr_linear* ws[1] = {&lw.o};
      if (int r = upload_group(c, ws, 1, 0, ly.o, true)) return r;
      const ifr_linear* wd[1] = {&lw.down};
      if (int r = upload_group(c, wd, 1, 0, ly.down, true)) return r;
    }
    if (lw.gate.bits == lw.up.bits && post_of(lw.gate) == post_of(lw.up)) {
      const ifr_linear* ws[2] = {&lw.gate, &lw.up};
      ly.ngu = 1;
      if (int r = upload_group(c, ws, 2, 1, ly.gu[0], true)) return r;
    } else {
      ly.ngu = 2;
      const ifr_linear* g1[1] = {&lw.gate};
      const ifr_linear* u1[1] = {&lw.up};
      if (int r = upload_group(c, g1, 1, 0, ly.gu[0], true)) return r;
      if (int r = upload_group(c, u1, 1, 0, ly.gu[1], true)) return r;
    }
    if (int r = upload(c, &ly.in_ln, lw.in_ln, H)) return r;
    if (int r = upload(c, &ly.post_ln, lw.post_ln, H)) return r;
    if (cf.qk_norm) {
      if (int r = upload(c, &ly.q_norm, lw.q_norm, hd)) return r;
      if (int r = upload(c, &ly.k_norm, lw.k_norm, hd)) return r;
    }
  }
  if (int r = upload(c, &c->embed, m->embed, (size_t)V * H)) return r;
  if (int r = upload(c, &c->final_norm, m->final_norm, H)) return r;
  // lm_head: per-row symmetric int8 of the output projection, the tied
  // embedding unless the model has its own (main.cpp:1745-1761).
  {
    const float* lmw = m->lm_head ? m->lm_head : m->embed;
    std::vector<uint8_t> q((size_t)V * H);
    std::vector<uint16_t> s(V);
    for (int r = 0; r < V; ++r) {
      const float* Wr = lmw + (size_t)r * H;
      float mx = 0;
      for (int k = 0; k < H; ++k) mx = std::max(mx, std::fabs(Wr[k]));
      const float sc = (mx > 0) ? mx / 127.0f : 1.0f;
      s[r] = ifr::f2h(sc);
      const float inv = 1.0f / sc;
      for (int k = 0; k < H; ++k) q[(size_t)r * H + k] = (uint8_t)(int8_t)std::lrint(Wr[k] * inv);
    }
    std::vector<uint32_t> packed((size_t)V * H / 4);
    ifrk::pack_linear_host(q.data(), nullptr, nullptr, V, H, 8, packed.data(), nullptr, 1, 0, 0u);
    if (int r = upload(c, &c->lm_w, packed.data(), packed.size())) return r;
    if (int r = upload(c, &c->lm_s, s.data(), s.size())) return r;
  }
  // RoPE tables: cos/sin(inv_freq[d] * pos) in fp32 (main.cpp:365-373, :10594-10596).
  {
    const int half = cf.rotary_dim / 2, P = kvc->max_seq_tokens;
    std::vector<float> inv(half), cs((size_t)P * half), sn((size_t)P * half);
    for (int d = 0; d < half; ++d)
      inv[d] = 1.0f / std::pow(cf.rope_theta, (2.0f * d) / (float)cf.rotary_dim);
    for (int p = 0; p < P; ++p)
      for (int d = 0; d < half; ++d) {
        const float f = inv[d] * (float)p;
        cs[(size_t)p * half + d] = std::cos(f);
        sn[(size_t)p * half + d] = std::sin(f);
      }
    if (int r = upload(c, &c->rope_cos, cs.data(), cs.size())) return r;
    if (int r = upload(c, &c->rope_sin, sn.data(), sn.size())) return r;
  }
  // paged KV pool (zero-filled so unused page slots stay finite)
  c->n_pages = kvc->pool_tokens / kPage;
  c->max_pages = (kvc->max_seq_tokens + kPage - 1) / kPage;
  const size_t esz = kvc->kv_int8 ? 1 : 2;
  const size_t page_bytes = (size_t)nkv * kPage * hd * esz;
  c->kpool.resize(L);
  c->vpool.resize(L);
  c->kscale.assign(L, nullptr);
  c->vscale.assign(L, nullptr);
  for (int l = 0; l < L; ++l) {
    c->kpool[l] = c->dalloc(page_bytes * c->n_pages);
    c->vpool[l] = c->dalloc(page_bytes * c->n_pages);
    if (!c->kpool[l] || !c->vpool[l]) return fail(IFR_ENOMEM, "KV pool (%zu B/layer)", 2 * page_bytes * c->n_pages);
    HIPCHK(hipMemsetAsync(c->kpool[l], 0, page_bytes * c->n_pages, c->st));
    HIPCHK(hipMemsetAsync(c->vpool[l], 0, page_bytes * c->n_pages, c->st));
    if (kvc->kv_int8) {
      const size_t sb = (size_t)nkv * kPage * 2 * c->n_pages;
      c->kscale[l] = static_cast<uint16_t*>(c->dalloc(sb));
      c->vscale[l] = static_cast<uint16_t*>(c->dalloc(sb));
      if (!c->kscale[l] || !c->vscale[l]) return fail(IFR_ENOMEM, "KV scales");
      HIPCHK(hipMemsetAsync(c->kscale[l], 0, sb, c->st));
      HIPCHK(hipMemsetAsync(c->vscale[l], 0, sb, c->st));
    }
  }
  {
    std::vector<void*> pools;
    for (int l = 0; l < L; ++l) {
      pools.push_back(c->kpool[l]);
      pools.push_back(c->vpool[l]);
      if (kvc->kv_int8) {
        pools.push_back(c->kscale[l]);
        pools.push_back(c->vscale[l]);
      }
    }
    c->npools = (int)pools.size();
    if (int r = upload(c, &c->pools_d, pools.data(), pools.size())) return r;
    if (int r = walloc(c, &c->copy_idx_d, (size_t)2 * c->max_pages)) return r;
  }
  c->free_pages.clear();
  for (int p = c->n_pages - 1; p >= 0; --p) c->free_pages.push_back(p);
  c->seqs.assign(kvc->max_seqs, Seq());
  const size_t btn = (size_t)kvc->max_seqs * c->max_pages;
  HIPCHK(hipHostMalloc(reinterpret_cast<void**>(&c->bt_h), btn * sizeof(int32_t), hipHostMallocDefault));
  std::memset(c->bt_h, 0, btn * sizeof(int32_t));
  if (int r = walloc(c, &c->bt_d, btn)) return r;
  HIPCHK(hipMemcpyAsync(c->bt_d, c->bt_h, btn * sizeof(int32_t), hipMemcpyHostToDevice, c->st));
  // workspaces, one set per lane
  const int Mx = kvc->max_rows;
  c->maxM = Mx;
  c->max_units = max_units_for(*kvc, nkv, c->qb);
  const int Kmax = std::max(std::max(H, qN), F);
  const int nparts = ifrk::lmhead_nparts(V);
  // lane 1 runs only when two lanes are configured
  for (int li = 0; li < (kvc->lanes == 2 ? 2 : 1); ++li) {
    Lane& L = c->lane[li];
    HIPCHK(hipHostMalloc(reinterpret_cast<void**>(&L.rows_h), (size_t)Mx * 5 * sizeof(int32_t), hipHostMallocDefault));
    HIPCHK(hipHostMalloc(reinterpret_cast<void**>(&L.best_h), (size_t)Mx * sizeof(int32_t), hipHostMallocDefault));
    int r = 0;
    if ((r = walloc(c, &L.rows_d, (size_t)Mx * 5)) || (r = walloc(c, &L.resid, (size_t)Mx * H)) ||
        (r = walloc(c, &L.aq, ifrk::atile_bytes(Mx, Kmax))) || (r = walloc(c, &L.as, (size_t)Mx)) ||
        (r = walloc(c, &L.gs, (size_t)Mx * (Kmax / 128))) ||
        (r = walloc(c, &L.qkv, (size_t)Mx * ((cf.attn_gate ? 2 * qN : qN) + 2 * kvN))) ||
        (cf.attn_gate && (r = walloc(c, &L.gate, (size_t)Mx * qN))) ||
        (r = walloc(c, &L.qbuf, (size_t)Mx * qN)) || (r = walloc(c, &L.y, (size_t)Mx * H)) ||
        (r = walloc(c, &L.mg, (size_t)Mx * F)) || (r = walloc(c, &L.gu, (size_t)Mx * 2 * F)) ||
        (r = walloc(c, &L.pk.cu_seqlens, (size_t)Mx + 1)) || (r = walloc(c, &L.pk.row_grp, Mx)) ||
        (r = walloc(c, &L.pk.row_seq, Mx)) || (r = walloc(c, &L.pk.row_pos, Mx)) ||
        (r = walloc(c, &L.pk.row_kind, Mx)) || (r = walloc(c, &L.pk.comb_base, Mx)) ||
        (r = walloc(c, &L.pk.comb_nsplit, Mx)) || (r = walloc(c, &L.pk.comb_tok, Mx)) ||
        (r = walloc(c, &L.pk.want_rows, Mx)) || (r = walloc(c, &L.row_tok, Mx)) ||
        (r = walloc(c, &L.lm_aq, ifrk::atile_bytes(Mx, H))) || (r = walloc(c, &L.lm_as, (size_t)Mx * (H / 64))) ||
        (r = walloc(c, &L.best_d, Mx)) || (r = walloc(c, &L.lm_pv, (size_t)nparts * Mx)) ||
        (r = walloc(c, &L.lm_pi, (size_t)nparts * Mx)) || (r = walloc(c, &L.pk.units, c->max_units)) ||
        (r = walloc(c, &L.pk.order, 4 * (size_t)c->max_units)) ||
        (r = walloc(c, &L.part_o, (size_t)c->max_units * 16 * kAttnTiles * hd)) ||
        (r = walloc(c, &L.part_ml, (size_t)c->max_units * 16 * kAttnTiles * 2)))
      return r;
    L.pk.row_tok = L.row_tok;
  }
  HIPCHK(hipStreamSynchronize(c->st));
  c->loaded = true;
  return IFR_OK;
}

// ---- sequences ---------------------------------------------------------------------

int ifr_seq_open(ifr_ctx* c, int32_t* slot) {
  if (!c || !slot) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  for (size_t i = 0; i < c->seqs.size(); ++i)
    if (!c->seqs[i].open) {
      c->seqs[i] = Seq();
      c->seqs[i].open = true;
      *slot = (int32_t)i;
      return IFR_OK;
    }
  return fail(IFR_ENOMEM, "all %zu sequence slots in use", c->seqs.size());
}

int ifr_seq_truncate(ifr_ctx* c, int32_t slot, int32_t len) {
  if (!c || !c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (slot < 0 || slot >= (int)c->seqs.size() || !c->seqs[slot].open) return fail(IFR_EINVAL, "slot %d", slot);
  Seq& s = c->seqs[slot];
  if (len < 0 || len > s.len) return fail(IFR_EINVAL, "truncate %d > len %d", len, s.len);
  const int keep = (len + kPage - 1) / kPage;
  while ((int)s.pages.size() > keep) {
    c->free_pages.push_back(s.pages.back());
    s.pages.pop_back();
  }
  s.len = len;
  return IFR_OK;
}

int ifr_seq_close(ifr_ctx* c, int32_t slot) {
  if (int r = ifr_seq_truncate(c, slot, 0)) return r;
  c->seqs[slot].open = false;
  return IFR_OK;
}

int ifr_seq_copy_prefix(ifr_ctx* c, int32_t dst, int32_t src, int32_t len) {
  if (!c || !c->loaded) return fail(IFR_ESTATE, "no model loaded");
  const int ns = (int)c->seqs.size();
  if (dst < 0 || dst >= ns || !c->seqs[dst].open) return fail(IFR_EINVAL, "slot %d", dst);
  if (src < 0 || src >= ns || !c->seqs[src].open || src == dst) return fail(IFR_EINVAL, "slot %d", src);
  Seq& d = c->seqs[dst];
  const Seq& sq = c->seqs[src];
  if (d.len != 0) return fail(IFR_ESTATE, "sequence %d is not empty", dst);
  if (len < 0 || len > sq.len) return fail(IFR_EINVAL, "prefix %d > length %d", len, sq.len);
  if (len == 0) return IFR_OK;
  const int need = (len + kPage - 1) / kPage;
  if (need > (int)c->free_pages.size()) return fail(IFR_ENOMEM, "KV pool exhausted");
  std::vector<int32_t> idx((size_t)2 * need);
  for (int i = 0; i < need; ++i) {
    const int p = c->free_pages.back();
    c->free_pages.pop_back();
    c->bt_h[(size_t)dst * c->max_pages + i] = p;
    d.pages.push_back(p);
    idx[i] = sq.pages[i];
    idx[need + i] = p;
  }
  HIPCHK(hipSetDevice(c->device));
  // the context stream is in order: the copy lands before any later forward
  HIPCHK(hipMemcpyAsync(c->bt_d + (size_t)dst * c->max_pages, c->bt_h + (size_t)dst * c->max_pages,
                        c->max_pages * sizeof(int32_t), hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(c->copy_idx_d, idx.data(), idx.size() * sizeof(int32_t), hipMemcpyHostToDevice,
                        c->st));
  const size_t esz = c->kv.kv_int8 ? 1 : 2;
  ifrk::PageCopyArgs a{};
  a.pools = c->pools_d;
  a.npools = c->npools;
  a.per = c->kv.kv_int8 ? 4 : 2;
  a.page_bytes[0] = a.page_bytes[1] = (size_t)c->cfg.n_kv * kPage * c->cfg.head_dim * esz;
  a.page_bytes[2] = a.page_bytes[3] = (size_t)c->cfg.n_kv * kPage * 2;
  a.sp = c->copy_idx_d;
  a.dp = c->copy_idx_d + need;
  a.n = need;
  HIPCHK(ifrk::launch_copy_pages(a, c->st));
  // idx is a host temporary: wait for the staged copies before it goes
  HIPCHK(hipStreamSynchronize(c->st));
  d.len = len;
  return IFR_OK;
}

int ifr_seq_len(ifr_ctx* c, int32_t slot, int32_t* len) {
  if (!c || !c->loaded || !len) return fail(IFR_ESTATE, "no model loaded");
  if (slot < 0 || slot >= (int)c->seqs.size() || !c->seqs[slot].open) return fail(IFR_EINVAL, "slot %d", slot);
  *len = c->seqs[slot].len;
  return IFR_OK;
}

int ifr_model_info(ifr_ctx* c, ifr_model_cfg* out) {
  if (!c || !out) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  *out = c->cfg;
  return IFR_OK;
}

int ifr_kv_capacity(ifr_ctx* c, int32_t* tokens) {
  if (!c || !c->loaded || !tokens) return fail(IFR_ESTATE, "no model loaded");
  *tokens = c->kv.max_seq_tokens;
  return IFR_OK;
}

int ifr_seq_load_kv(ifr_ctx* c, int32_t slot, int32_t len, const float* k, const float* v) {
  if (!c || !c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (slot < 0 || slot >= (int)c->seqs.size() || !c->seqs[slot].open) return fail(IFR_EINVAL, "slot %d", slot);
  Seq& s = c->seqs[slot];
  if (s.len != 0) return fail(IFR_ESTATE, "sequence %d is not empty", slot);
  if (len < 0 || len > c->kv.max_seq_tokens || !k || !v) return fail(IFR_EINVAL, "len %d", len);
  const int need = (len + kPage - 1) / kPage;
  if (need > (int)c->free_pages.size()) return fail(IFR_ENOMEM, "KV pool exhausted");
  for (int i = 0; i < need; ++i) {
    const int p = c->free_pages.back();
    c->free_pages.pop_back();
    c->bt_h[(size_t)slot * c->max_pages + i] = p;
    s.pages.push_back(p);
  }
  HIPCHK(hipMemcpy(c->bt_d + (size_t)slot * c->max_pages, c->bt_h + (size_t)slot * c->max_pages,
                   c->max_pages * sizeof(int32_t), hipMemcpyHostToDevice));
  const int nkv = c->cfg.n_kv, hd = c->cfg.head_dim, L = c->cfg.layers;
  const bool i8 = c->kv.kv_int8 != 0;
  const size_t per_page = (size_t)nkv * kPage * hd;
  std::vector<uint16_t> kh(per_page), vh(per_page), ksc((size_t)nkv * kPage), vsc((size_t)nkv * kPage);
  std::vector<int8_t> kq(per_page), vq(per_page);
  // One (token, head) vector: fp16 round, then optionally int8 (same rule as
  // the kernel); element d goes to block index off(d) (kv_koff / kv_voff order).
  auto enc = [&](const float* x, uint16_t* h16, int8_t* q8, uint16_t* sc, auto off) {
    float r[128];
    float mx = 0;
    for (int d = 0; d < hd; ++d) {
      r[d] = ifr::h2f(ifr::f2h(x[d]));
      mx = std::max(mx, std::fabs(r[d]));
    }
    if (!i8) {
      for (int d = 0; d < hd; ++d) h16[off(d)] = ifr::f2h(r[d]);
      return;
    }
    const uint16_t s16 = ifr::f2h(mx > 0 ? mx / 127.0f : 1.0f);
    const float inv = 1.0f / ifr::h2f(s16);
    for (int d = 0; d < hd; ++d) {
      const float t = r[d] * inv;
      int q = (int)(t >= 0.0f ? t + 0.5f : t - 0.5f);
      q = std::min(127, std::max(-127, q));
      q8[off(d)] = (int8_t)q;
    }
    *sc = s16;
  };
  for (int l = 0; l < L; ++l) {
    for (int pi = 0; pi < need; ++pi) {
      std::fill(kh.begin(), kh.end(), 0);
      std::fill(vh.begin(), vh.end(), 0);
      std::fill(kq.begin(), kq.end(), 0);
      std::fill(vq.begin(), vq.end(), 0);
      std::fill(ksc.begin(), ksc.end(), 0);
      std::fill(vsc.begin(), vsc.end(), 0);
      for (int tk = 0; tk < kPage; ++tk) {
        const int t = pi * kPage + tk;
        if (t >= len) break;
        for (int h = 0; h < nkv; ++h) {
          const size_t src = (((size_t)l * len + t) * nkv + h) * hd;
          const size_t blk = (size_t)h * kPage * hd;  // this head's 32 x 128 block
          enc(k + src, &kh[blk], &kq[blk], &ksc[(size_t)h * kPage + tk],
              [&](int d) { return ifrk::kv_koff(tk, d); });
          enc(v + src, &vh[blk], &vq[blk], &vsc[(size_t)h * kPage + tk],
              [&](int d) { return ifrk::kv_voff(tk, d); });
        }
      }
      const size_t page = (size_t)s.pages[pi];
      if (!i8) {
        HIPCHK(hipMemcpy(static_cast<uint16_t*>(c->kpool[l]) + page * per_page, kh.data(), per_page * 2, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(static_cast<uint16_t*>(c->vpool[l]) + page * per_page, vh.data(), per_page * 2, hipMemcpyHostToDevice));
      } else {
        HIPCHK(hipMemcpy(static_cast<int8_t*>(c->kpool[l]) + page * per_page, kq.data(), per_page, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(static_cast<int8_t*>(c->vpool[l]) + page * per_page, vq.data(), per_page, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(c->kscale[l] + page * nkv * kPage, ksc.data(), ksc.size() * 2, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(c->vscale[l] + page * nkv * kPage, vsc.data(), vsc.size() * 2, hipMemcpyHostToDevice));
      }
    }
  }
  s.len = len;
  return IFR_OK;
}

// ---- forward ---------------------------------------------------------------------------

int ifr_forward(ifr_ctx* c, const ifr_row* rows, int32_t M, int32_t* best_out, float* logits_out) {
  const auto t_start = std::chrono::steady_clock::now();
  if (!c || !rows || !best_out) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (M <= 0 || M > c->maxM) return fail(IFR_EINVAL, "M=%d outside [1, %d]", M, c->maxM);
  const int V = c->cfg.vocab;
  // ---- validate rows (BatchItem rules: one contiguous run per sequence)
  std::vector<int> g_start, g_len, g_pos0, g_seq;
  bool any_logit_rows = false;  // logits_out then holds only the want = 2 rows
  for (int m = 0; m < M; ++m) {
    const ifr_row& r = rows[m];
    if (r.seq < 0 || r.seq >= (int)c->seqs.size() || !c->seqs[r.seq].open)
      return fail(IFR_EINVAL, "row %d: sequence slot %d not open", m, r.seq);
    if (r.token < 0 || r.token >= V) return fail(IFR_EINVAL, "row %d: token %d", m, r.token);
    if (r.kind < IFR_ROW_DECODE || r.kind > IFR_ROW_VERIFY) return fail(IFR_EINVAL, "row %d: kind", m);
    if (r.want < 0 || r.want > 2) return fail(IFR_EINVAL, "row %d: want %d", m, r.want);
    if (r.want == 2) any_logit_rows = true;
    if (r.pos < 0 || r.pos >= c->kv.max_seq_tokens)
      return fail(IFR_EINVAL, "row %d: pos %d >= KV capacity %d", m, r.pos, c->kv.max_seq_tokens);
    const bool first = (m == 0 || rows[m - 1].seq != r.seq);
    if (first) {
      if (r.pos != c->seqs[r.seq].len)
        return fail(IFR_EINVAL, "row %d: pos %d != sequence length %d", m, r.pos, c->seqs[r.seq].len);
      for (int s : g_seq)
        if (s == r.seq) return fail(IFR_EINVAL, "row %d: sequence %d appears twice", m, r.seq);
      g_start.push_back(m);
      g_len.push_back(1);
      g_pos0.push_back(r.pos);
      g_seq.push_back(r.seq);
    } else {
      if (r.pos != rows[m - 1].pos + 1) return fail(IFR_EINVAL, "row %d: positions not consecutive", m);
      g_len.back() += 1;
    }
  }
  // ---- pages for every new position (block table rows go up on lane 0);
  // checked for the whole batch first, so a refusal changes nothing
  {
    size_t more = 0;
    for (size_t g = 0; g < g_seq.size(); ++g) {
      const Seq& s = c->seqs[g_seq[g]];
      const int need = (g_pos0[g] + g_len[g] + kPage - 1) / kPage;
      if (need > (int)s.pages.size()) more += (size_t)(need - (int)s.pages.size());
    }
    if (more > c->free_pages.size())
      return fail(IFR_ENOMEM, "KV pool exhausted (%zu pages needed, %zu free)", more, c->free_pages.size());
  }
  // new pages go into the pinned host block table; the rows of the
  // sequences that grew go up in one copy (their slot range)
  int dlo = INT32_MAX, dhi = -1;
  for (size_t g = 0; g < g_seq.size(); ++g) {
    Seq& s = c->seqs[g_seq[g]];
    const int need = (g_pos0[g] + g_len[g] + kPage - 1) / kPage;
    while ((int)s.pages.size() < need) {
      const int p = c->free_pages.back();
      c->free_pages.pop_back();
      c->bt_h[(size_t)g_seq[g] * c->max_pages + s.pages.size()] = p;
      s.pages.push_back(p);
      dlo = std::min(dlo, g_seq[g]);
      dhi = std::max(dhi, g_seq[g]);
    }
  }
  if (dhi >= 0) {
    const size_t off = (size_t)dlo * c->max_pages;
    HIPCHK(hipMemcpyAsync(c->bt_d + off, c->bt_h + off, (size_t)(dhi - dlo + 1) * c->max_pages * sizeof(int32_t),
                          hipMemcpyHostToDevice, c->lane[0].st));
  }
  // ---- cut into sub-batches: [decode / verify rows | prefill chunks], or
  // decode rows halved by KV length; one sub-batch when timing each kernel
  const int ng = (int)g_len.size();
  int cut = ng;  // first group of lane 1
  if (!c->timing && c->kv.lanes == 2 && ng >= 2) {
    int first_chunk = ng;
    for (int g = 0; g < ng; ++g)
      if (g_len[g] >= kChunkRows) { first_chunk = g; break; }
    if (first_chunk > 0 && first_chunk < ng) {
      cut = first_chunk;
    } else if (first_chunk == ng && M >= kMinSplitRows) {
      double tot = 0, run = 0;
      for (int g = 0; g < ng; ++g) tot += g_pos0[g] + g_len[g];
      for (cut = 0; cut < ng - 1 && run + 0.5 * (g_pos0[cut] + g_len[cut]) < 0.5 * tot; ++cut)
        run += g_pos0[cut] + g_len[cut];
      if (cut == 0) cut = 1;
    }
  }
  std::vector<SubBatch> sbs;
  for (int h = 0; h < 2; ++h) {
    const int ga = h == 0 ? 0 : cut, gb = h == 0 ? cut : ng;
    if (ga >= gb) continue;
    SubBatch sb;
    sb.lane = h;
    sb.row0 = g_start[ga];
    sb.M = (gb < ng ? g_start[gb] : M) - sb.row0;
    sb.g_pos0.assign(g_pos0.begin() + ga, g_pos0.begin() + gb);
    sb.g_len.assign(g_len.begin() + ga, g_len.begin() + gb);
    if (int r = prep_sub(c, rows, sb)) return r;
    sbs.push_back(std::move(sb));
  }
  c->last_lanes = (int)sbs.size();
  if (sbs.size() == 2) {
    HIPCHK(hipEventRecord(c->ev_bt, c->lane[0].st));
    HIPCHK(hipStreamWaitEvent(c->lane[1].st, c->ev_bt, 0));
  }
  // ---- enqueue: heads, then layer by layer alternating lanes, then tails
  for (SubBatch& sb : sbs)
    if (int r = launch_head(c, rows, sb)) return r;
  for (int l = 0; l < c->cfg.layers; ++l)
    for (SubBatch& sb : sbs)
      if (int r = launch_layer(c, sb, l)) return r;
  int want_off = 0;
  for (SubBatch& sb : sbs) {
    if (int r = launch_tail(c, sb, logits_out ? logits_out + (size_t)want_off * V : nullptr, any_logit_rows))
      return r;
    want_off += (int)(any_logit_rows ? sb.want_logits.size() : sb.want.size());
  }
  const auto t_sub = std::chrono::steady_clock::now();
  for (SubBatch& sb : sbs) HIPCHK(hipStreamSynchronize(c->lane[sb.lane].st));
  const auto t_end = std::chrono::steady_clock::now();
  // host buckets (the reference engine's submit / waitblock profile,
  // engine.hpp:567-630), kept whether or not kernels are timed
  add_host_time(c, "host_submit", std::chrono::duration<double, std::milli>(t_sub - t_start).count());
  add_host_time(c, "host_wait", std::chrono::duration<double, std::milli>(t_end - t_sub).count());
  for (int m = 0; m < M; ++m) best_out[m] = -1;
  for (const SubBatch& sb : sbs)
    for (size_t i = 0; i < sb.want.size(); ++i) best_out[sb.row0 + sb.want[i]] = c->lane[sb.lane].best_h[i];
  for (size_t g = 0; g < g_seq.size(); ++g) c->seqs[g_seq[g]].len = g_pos0[g] + g_len[g];
  if (c->timing) flush_timers(c);
  return IFR_OK;
}

}  // extern "C"

namespace {

// Rows of an attention-only call: open sequences whose KV already holds every
// row's position, one contiguous run of consecutive positions per sequence.
int attn_groups(ifr_ctx* c, const ifr_row* rows, int M, std::vector<int>& g_len, std::vector<int>& g_pos0) {
  std::vector<int> g_seq;
  for (int m = 0; m < M; ++m) {
    const ifr_row& r = rows[m];
    if (r.seq < 0 || r.seq >= (int)c->seqs.size() || !c->seqs[r.seq].open)
      return fail(IFR_EINVAL, "row %d: sequence slot %d not open", m, r.seq);
    if (r.pos < 0 || r.pos >= c->seqs[r.seq].len)
      return fail(IFR_EINVAL, "row %d: pos %d has no KV (len %d)", m, r.pos, c->seqs[r.seq].len);
    const bool first = (m == 0 || rows[m - 1].seq != r.seq);
    if (first) {
      for (int s : g_seq)
        if (s == r.seq) return fail(IFR_EINVAL, "row %d: sequence %d appears twice", m, r.seq);
      g_len.push_back(1);
      g_pos0.push_back(r.pos);
      g_seq.push_back(r.seq);
    } else {
      if (r.pos != rows[m - 1].pos + 1) return fail(IFR_EINVAL, "row %d: positions not consecutive", m);
      g_len.back() += 1;
    }
  }
  return IFR_OK;
}

}  // namespace

extern "C" {

int ifr_attention(ifr_ctx* c, int32_t layer, const ifr_row* rows, int32_t M, const uint16_t* q_h,
                  float* out_h) {
  if (!c || !rows || !q_h || !out_h) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (M <= 0 || M > c->maxM) return fail(IFR_EINVAL, "M=%d outside [1, %d]", M, c->maxM);
  if (layer < 0 || layer >= c->cfg.layers) return fail(IFR_EINVAL, "layer %d", layer);
  const int nq = c->cfg.n_heads, nkv = c->cfg.n_kv, hd = c->cfg.head_dim;
  std::vector<int> g_len, g_pos0;
  if (int r = attn_groups(c, rows, M, g_len, g_pos0)) return r;
  const int split = c->kv.attn_split > 0 ? c->kv.attn_split : kSplit;
  const long nunits = count_units(g_pos0, g_len, nkv, split, c->qb);
  if (nunits > c->max_units)
    return fail(IFR_EDECLINE, "batch needs %ld attention units, the workspace holds %d (KV split %d)", nunits,
                c->max_units, split);
  c->last_split = split;
  c->last_units = (int)nunits;
  long nchunked = 0;
  const int nslots = (int)ifrk::attn_slot_count(g_pos0.data(), g_len.data(), (int)g_len.size(), nkv, split,
                                                c->qb, &nchunked);
  c->last_slots = nslots;
  std::memcpy(c->lane[0].rows_h, rows, (size_t)M * sizeof(ifr_row));
  HIPCHK(hipMemcpyAsync(c->lane[0].rows_d, c->lane[0].rows_h, (size_t)M * sizeof(ifr_row), hipMemcpyHostToDevice, c->st));
  HIPCHK(ifrk::launch_pack(c->lane[0].rows_d, M, nkv, c->qb, split, c->lane[0].pk, c->st));
  HIPCHK(hipMemcpyAsync(c->lane[0].qbuf, q_h, (size_t)M * nq * hd * 2, hipMemcpyHostToDevice, c->st));
  ifrk::KVLayout kv{nkv, hd, kPage, c->max_pages, c->kv.kv_int8, c->kpool[layer], c->vpool[layer],
                    c->kscale[layer], c->vscale[layer], c->bt_d};
  ifrk::AttnArgs a{c->lane[0].pk.units, (int)nunits, c->lane[0].pk.order, nslots, shared_slots(c, nchunked), c->lane[0].qbuf, nq, 1.4426950408889634f / std::sqrt((float)hd),
                   c->lane[0].part_o, c->lane[0].part_ml, kAttnTiles};
  double attn_bytes = 0, attn_flops = 0;
  attn_work(c, rows, M, g_pos0, g_len, &attn_bytes, &attn_flops);
  {
    Scope sc(c, c->st, "attention", attn_bytes, attn_flops);
    HIPCHK(ifrk::launch_attention(a, kv, c->st));
  }
  float* out_d = nullptr;
  HIPCHK(hipMalloc(reinterpret_cast<void**>(&out_d), (size_t)M * nq * hd * sizeof(float)));
  ifrk::CombineArgs cb{c->lane[0].part_o, c->lane[0].part_ml, c->lane[0].pk.comb_base, c->lane[0].pk.comb_nsplit, c->lane[0].pk.comb_tok,
                       M, nq, nkv, hd, out_d, c->lane[0].aq, c->lane[0].as, c->lane[0].gs, 16 * kAttnTiles};
  hipError_t e;
  {
    Scope sc(c, c->st, "combine", combine_work(c, M, g_pos0, g_len, split, c->qb));
    e = ifrk::launch_combine(cb, c->st);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(out_h, out_d, (size_t)M * nq * hd * sizeof(float), hipMemcpyDeviceToHost, c->st);
  if (e == hipSuccess) e = hipStreamSynchronize(c->st);
  hipFree(out_d);
  HIPCHK(e);
  if (c->timing) flush_timers(c);
  return IFR_OK;
}

int ifr_attention_noalloc(ifr_ctx* c, int32_t layer, const ifr_row* rows, int32_t M, const uint16_t* q_d,
                          float* out_d) {
  if (!c || !rows || !q_d || !out_d) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (!c->scratch) return fail(IFR_ESTATE, "scratch address not resolved");
  if (M <= 0 || M > kNaRows) return fail(IFR_EINVAL, "M=%d outside [1, %d] (no-allocation limit)", M, kNaRows);
  if (layer < 0 || layer >= c->cfg.layers) return fail(IFR_EINVAL, "layer %d", layer);
  const int nq = c->cfg.n_heads, nkv = c->cfg.n_kv, hd = c->cfg.head_dim;
  if (nq * hd > kNaRowWidth) return fail(IFR_EINVAL, "n_heads * head_dim %d > %d", nq * hd, kNaRowWidth);
  std::vector<int> g_len, g_pos0;
  if (int r = attn_groups(c, rows, M, g_len, g_pos0)) return r;
  // the engine's split, never widened here: a batch that needs more units
  // than the scratch holds is refused instead
  const int split = c->kv.attn_split > 0 ? c->kv.attn_split : kSplit;
  const long nunits = count_units(g_pos0, g_len, nkv, split, c->qb);
  long nchunked = 0;
  const long nslots = ifrk::attn_slot_count(g_pos0.data(), g_len.data(), (int)g_len.size(), nkv, split, c->qb,
                                            &nchunked);
  if (nunits > kNaUnits || nslots > 4L * kNaUnits)
    return fail(IFR_EINVAL, "%ld attention units (%ld slots) > %d (no-allocation limit)", nunits, nslots, kNaUnits);
  HIPCHK(hipSetDevice(c->device));
  std::lock_guard<std::mutex> hold(g_na_lock[c->device % kNaLockDevices]);
  uint8_t* S = c->scratch;
  int32_t* rows_d = reinterpret_cast<int32_t*>(S + kNaRowsOff);
  auto map = [&](int i) { return reinterpret_cast<int32_t*>(S + kNaMapsOff + (size_t)i * kNaMapLen); };
  ifrk::PackOut pk{};
  pk.cu_seqlens = map(0);
  pk.row_grp = map(1);
  pk.row_seq = map(2);
  pk.row_pos = map(3);
  pk.row_kind = map(4);
  pk.comb_base = map(5);
  pk.comb_nsplit = map(6);
  pk.comb_tok = map(7);
  pk.want_rows = map(8);
  pk.units = reinterpret_cast<ifrk::AttnUnit*>(S + kNaUnitsOff);
  pk.order = reinterpret_cast<int32_t*>(S + kNaOrderOff);
  float* part_o = reinterpret_cast<float*>(S + kNaPartOOff);
  float* part_ml = reinterpret_cast<float*>(S + kNaPartMLOff);
  // every region is fully written by the kernel that produces it before it
  // is read (the pack maps, each unit's partials, the combine outputs), so
  // nothing is cleared between calls
  HIPCHK(hipMemcpyAsync(rows_d, rows, (size_t)M * sizeof(ifr_row), hipMemcpyHostToDevice, c->st));
  HIPCHK(ifrk::launch_pack(rows_d, M, nkv, c->qb, split, pk, c->st));
  ifrk::KVLayout kv{nkv, hd, kPage, c->max_pages, c->kv.kv_int8, c->kpool[layer], c->vpool[layer],
                    c->kscale[layer], c->vscale[layer], c->bt_d};
  ifrk::AttnArgs a{pk.units, (int)nunits, pk.order, (int)nslots, shared_slots(c, nchunked), q_d, nq,
                   1.4426950408889634f / std::sqrt((float)hd), part_o, part_ml, kAttnTiles};
  HIPCHK(ifrk::launch_attention(a, kv, c->st));
  ifrk::CombineArgs cb{part_o, part_ml, pk.comb_base, pk.comb_nsplit, pk.comb_tok, M, nq, nkv, hd, out_d,
                       reinterpret_cast<int8_t*>(S + kNaAqOff), reinterpret_cast<float*>(S + kNaAsOff),
                       reinterpret_cast<float*>(S + kNaGsOff), 16 * kAttnTiles};
  HIPCHK(ifrk::launch_combine(cb, c->st));
  // the rows copy read the caller's host array; return once out_d is written
  HIPCHK(hipStreamSynchronize(c->st));
  return IFR_OK;
}

}  // extern "C"

namespace {

// Widest input (K) and output (N) of any linear of the loaded model.
void seam_dims(const ifr_ctx* c, int* Kmax, int* Nmax) {
  const ifr_model_cfg& cf = c->cfg;
  const int qN = cf.n_heads * cf.head_dim, qrows = (cf.attn_gate ? 2 : 1) * qN, kvN = cf.n_kv * cf.head_dim;
  *Kmax = std::max(std::max(cf.hidden, qN), cf.inter);
  *Nmax = std::max(std::max(qrows + 2 * kvN, 2 * cf.inter), cf.hidden);
}

int seam_alloc(ifr_ctx* c) {
  if (c->sx) return IFR_OK;
  int Kmax = 0, Nmax = 0;
  seam_dims(c, &Kmax, &Nmax);
  const size_t Mx = (size_t)c->maxM;
  int r = 0;
  if ((r = walloc(c, &c->sx, Mx * Kmax)) || (r = walloc(c, &c->saq, ifrk::atile_bytes((int)Mx, Kmax))) ||
      (r = walloc(c, &c->sas, Mx)) || (r = walloc(c, &c->sgs, Mx * (Kmax / 128))) ||
      (r = walloc(c, &c->sy, Mx * Nmax)) || (r = walloc(c, &c->smg, Mx * c->cfg.inter))) {
    c->sx = nullptr;
    return r;
  }
  return IFR_OK;
}

// The device linear of (layer, which) as the GEMM runs it.  Q, K and V of a
// fused QKV projection are its tile ranges (tiles are contiguous in the
// fragment-major layout); gate and up of an interleaved pair are the pair
// run as a plain GEMM (tiles gate 0, up 0, gate 1, ...), *deint = 1 (gate)
// or 2 (up) picking its tiles out of that output.
int seam_view(ifr_ctx* c, int layer, int which, DLin& v, int* deint) {
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (layer < 0 || layer >= c->cfg.layers) return fail(IFR_EINVAL, "layer %d", layer);
  const ifr_model_cfg& cf = c->cfg;
  const int qrows = (cf.attn_gate ? 2 : 1) * cf.n_heads * cf.head_dim, kvN = cf.n_kv * cf.head_dim;
  const Layer& ly = c->layers[layer];
  *deint = 0;
  switch (which) {
    case IFR_LIN_Q:
    case IFR_LIN_K:
    case IFR_LIN_V: {
      if (ly.nqkv == 3) {
        v = ly.qkv[which];
        return IFR_OK;
      }
      const int off = which == IFR_LIN_Q ? 0 : which == IFR_LIN_K ? qrows : qrows + kvN;
      v = ly.qkv[0];
      const size_t t0 = (size_t)off / 16;
      v.codes += t0 * v.nsteps * 64 * (v.bits / 2);
      v.sz += t0 * v.ng * 16;
      v.N = which == IFR_LIN_Q ? qrows : kvN;
      return IFR_OK;
    }
    case IFR_LIN_O: v = ly.o; return IFR_OK;
    case IFR_LIN_DOWN: v = ly.down; return IFR_OK;
    case IFR_LIN_GATE:
    case IFR_LIN_UP:
      if (ly.ngu == 2) {
        v = ly.gu[which - IFR_LIN_GATE];
      } else {
        v = ly.gu[0];
        v.pair = 0;
        *deint = 1 + (which - IFR_LIN_GATE);
      }
      return IFR_OK;
    default: return fail(IFR_EINVAL, "linear id %d", which);
  }
}

// Enqueue one linear over m rows already in c->sx: per-token quantization,
// the GEMM into c->sy, and the fp16 rows back into c->hy.
int seam_enqueue(ifr_ctx* c, const DLin& v, int m) {
  HIPCHK(ifrk::launch_quant_plain(c->sx, nullptr, m, v.K, c->saq, c->sas, c->sgs, c->st));
  ifrk::QGemmArgs a{c->saq, c->sas, c->sgs, c->sy, nullptr, m, v.N};
  HIPCHK(ifrk::launch_qgemm(v, a, c->st));
  return IFR_OK;
}

// fp16 rows [m][v.N] of the chunk into fp32 Y (de-interleaving a pair's tiles)
void seam_unpack(const ifr_ctx* c, const DLin& v, int deint, int m, float* Y) {
  const int Nout = deint ? v.N / 2 : v.N;
  for (int r = 0; r < m; ++r) {
    const uint16_t* src = c->hy.data() + (size_t)r * v.N;
    float* dst = Y + (size_t)r * Nout;
    if (!deint) {
      for (int n = 0; n < Nout; ++n) dst[n] = ifr::h2f(src[n]);
    } else {
      for (int n = 0; n < Nout; ++n) dst[n] = ifr::h2f(src[32 * (n / 16) + 16 * (deint - 1) + (n % 16)]);
    }
  }
}

// One linear over M host rows, in chunks of max_rows.
int seam_linear(ifr_ctx* c, int layer, int which, const float* X, float* Y, int M) {
  DLin v;
  int deint = 0;
  if (int r = seam_view(c, layer, which, v, &deint)) return r;
  if (int r = seam_alloc(c)) return r;
  const int Nout = deint ? v.N / 2 : v.N;
  c->hy.resize((size_t)c->maxM * v.N);
  for (int r0 = 0; r0 < M; r0 += c->maxM) {
    const int m = std::min(c->maxM, M - r0);
    HIPCHK(hipMemcpyAsync(c->sx, X + (size_t)r0 * v.K, (size_t)m * v.K * sizeof(float), hipMemcpyHostToDevice, c->st));
    if (int r = seam_enqueue(c, v, m)) return r;
    HIPCHK(hipMemcpyAsync(c->hy.data(), c->sy, (size_t)m * v.N * 2, hipMemcpyDeviceToHost, c->st));
    HIPCHK(hipStreamSynchronize(c->st));
    seam_unpack(c, v, deint, m, Y + (size_t)r0 * Nout);
  }
  return IFR_OK;
}

}  // namespace

extern "C" {

int ifr_linear_lookup(ifr_ctx* c, const char* name, int32_t* layer, int32_t* which) {
  if (!c || !name || !layer || !which) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  static const char* const kSuffix[7] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                         "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                                         "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                         "mlp.down_proj.weight"};
  const std::string n(name), pre = "model.language_model.layers.";
  if (n.compare(0, pre.size(), pre) != 0) return fail(IFR_EINVAL, "not a layer linear: %s", name);
  size_t i = pre.size(), j = i;
  while (j < n.size() && n[j] >= '0' && n[j] <= '9') ++j;
  if (j == i || j - i > 6 || j >= n.size() || n[j] != '.') return fail(IFR_EINVAL, "no layer index in %s", name);
  const int l = std::atoi(n.substr(i, j - i).c_str());
  if (l >= c->cfg.layers) return fail(IFR_EINVAL, "layer %d of %d in %s", l, c->cfg.layers, name);
  for (int w = 0; w < 7; ++w)
    if (n.compare(j + 1, std::string::npos, kSuffix[w]) == 0) {
      *layer = l;
      *which = w;
      return IFR_OK;
    }
  return fail(IFR_EINVAL, "not a linear of the model: %s", name);
}

int ifr_linear_shape(ifr_ctx* c, int32_t layer, int32_t which, int32_t* N, int32_t* K) {
  if (!c || !N || !K) return fail(IFR_EINVAL, "null arg");
  DLin v;
  int deint = 0;
  if (int r = seam_view(c, layer, which, v, &deint)) return r;
  *N = deint ? v.N / 2 : v.N;
  *K = v.K;
  return IFR_OK;
}

int ifr_linear_rot(ifr_ctx* c, int32_t which, int32_t* site) {
  if (!c || !site) return fail(IFR_EINVAL, "null arg");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (which < IFR_LIN_Q || which > IFR_LIN_DOWN) return fail(IFR_EINVAL, "linear id %d", which);
  *site = !c->cfg.rotate ? 0 : (which == IFR_LIN_O || which == IFR_LIN_DOWN) ? 2 : 1;
  return IFR_OK;
}

int ifr_linear_batch(ifr_ctx* c, int32_t layer, int32_t which, const float* X, float* Y, int32_t M) {
  if (!c || !X || !Y || M < 0) return fail(IFR_EINVAL, "null arg or M < 0");
  if (M == 0) return IFR_OK;
  HIPCHK(hipSetDevice(c->device));
  return seam_linear(c, layer, which, X, Y, M);
}

int ifr_linear_wave_batch(ifr_ctx* c, const ifr_linear_item* items, int32_t n, int32_t M) {
  if (!c || (n > 0 && !items) || n < 0 || M < 0) return fail(IFR_EINVAL, "null arg");
  HIPCHK(hipSetDevice(c->device));
  // items are independent: each one's rows run through the shared staging
  // in turn; the results equal ifr_linear_batch item by item
  for (int i = 0; i < n; ++i) {
    if (!items[i].X || !items[i].Y) return fail(IFR_EINVAL, "item %d: null buffer", i);
    if (M == 0) continue;
    if (int r = seam_linear(c, items[i].layer, items[i].which, items[i].X, items[i].Y, M)) return r;
  }
  return IFR_OK;
}

int ifr_mlp_fused(ifr_ctx* c, int32_t layer, const float* rin, float* md, int32_t M) {
  if (!c || !rin || !md || M < 0) return fail(IFR_EINVAL, "null arg or M < 0");
  if (!c->loaded) return fail(IFR_ESTATE, "no model loaded");
  if (layer < 0 || layer >= c->cfg.layers) return fail(IFR_EINVAL, "layer %d", layer);
  if (M == 0) return IFR_OK;
  HIPCHK(hipSetDevice(c->device));
  if (int r = seam_alloc(c)) return r;
  const ifr_model_cfg& cf = c->cfg;
  const int H = cf.hidden, F = cf.inter;
  const Layer& ly = c->layers[layer];
  c->hy.resize((size_t)c->maxM * H);
  for (int r0 = 0; r0 < M; r0 += c->maxM) {
    const int m = std::min(c->maxM, M - r0);
    HIPCHK(hipMemcpyAsync(c->sx, rin + (size_t)r0 * H, (size_t)m * H * sizeof(float), hipMemcpyHostToDevice, c->st));
    HIPCHK(ifrk::launch_quant_plain(c->sx, nullptr, m, H, c->saq, c->sas, c->sgs, c->st));
    // gate/up with the SwiGLU epilogue (or two GEMMs and the SwiGLU pass),
    // then the down projection's per-token quantization: the forward's steps
    if (ly.ngu == 1) {
      ifrk::QGemmArgs a{c->saq, c->sas, c->sgs, c->smg, nullptr, m, F};
      HIPCHK(ifrk::launch_qgemm(ly.gu[0], a, c->st));
    } else {
      for (int j = 0; j < 2; ++j) {
        ifrk::QGemmArgs a{c->saq, c->sas, c->sgs, c->sy + j * F, nullptr, m, 2 * F};
        HIPCHK(ifrk::launch_qgemm(ly.gu[j], a, c->st));
      }
      HIPCHK(ifrk::launch_swiglu(c->sy, m, F, c->smg, c->st));
    }
    HIPCHK(ifrk::launch_quant_plain(nullptr, c->smg, m, F, c->saq, c->sas, c->sgs, c->st));
    ifrk::QGemmArgs a{c->saq, c->sas, c->sgs, c->sy, nullptr, m, H};
    HIPCHK(ifrk::launch_qgemm(ly.down, a, c->st));
    HIPCHK(hipMemcpyAsync(c->hy.data(), c->sy, (size_t)m * H * 2, hipMemcpyDeviceToHost, c->st));
    HIPCHK(hipStreamSynchronize(c->st));
    for (size_t i = 0; i < (size_t)m * H; ++i) md[(size_t)r0 * H + i] = ifr::h2f(c->hy[i]);
  }
  return IFR_OK;
}

int ifr_set_timing(ifr_ctx* c, int32_t on) {
  if (!c) return fail(IFR_EINVAL, "ctx null");
  c->timing = on != 0;
  c->stats.clear();
  return IFR_OK;
}

int ifr_get_timing(ifr_ctx* c, const char* kernel, double* total_ms, int64_t* launches,
                   double* bytes, double* flops) {
  if (!c || !kernel) return fail(IFR_EINVAL, "null arg");
  for (auto& s : c->stats)
    if (s.first == kernel) {
      if (total_ms) *total_ms = s.second.ms;
      if (launches) *launches = s.second.n;
      if (bytes) *bytes = s.second.bytes;
      if (flops) *flops = s.second.flops;
      return IFR_OK;
    }
  if (total_ms) *total_ms = 0;
  if (launches) *launches = 0;
  if (bytes) *bytes = 0;
  if (flops) *flops = 0;
  return IFR_OK;
}

int ifr_debug_last_lanes(ifr_ctx* c, int32_t* lanes) {
  if (!c || !lanes) return fail(IFR_EINVAL, "null arg");
  *lanes = c->last_lanes;
  return IFR_OK;
}

int ifr_debug_attn_order(ifr_ctx* c, int32_t* order, int32_t cap, int32_t* n_slots) {
  if (!c || !n_slots) return fail(IFR_EINVAL, "null arg");
  HIPCHK(hipStreamSynchronize(c->st));
  *n_slots = c->last_slots;
  if (order && cap > 0)
    HIPCHK(hipMemcpy(order, c->lane[0].pk.order, (size_t)std::min(cap, c->last_slots) * 4, hipMemcpyDeviceToHost));
  return IFR_OK;
}

// Test hook: device pointers of the last forward's pack outputs.
int ifr_debug_pack(ifr_ctx* c, int32_t M, int32_t* cu, int32_t* row_grp, int32_t* comb_base,
                   int32_t* comb_nsplit, int32_t* comb_tok, int32_t* units, int32_t* n_units,
                   int32_t* split) {
  if (!c || !c->loaded) return fail(IFR_ESTATE, "no model loaded");
  HIPCHK(hipStreamSynchronize(c->st));
  if (cu) HIPCHK(hipMemcpy(cu, c->lane[0].pk.cu_seqlens, (M + 1) * 4, hipMemcpyDeviceToHost));
  if (row_grp) HIPCHK(hipMemcpy(row_grp, c->lane[0].pk.row_grp, M * 4, hipMemcpyDeviceToHost));
  if (comb_base) HIPCHK(hipMemcpy(comb_base, c->lane[0].pk.comb_base, M * 4, hipMemcpyDeviceToHost));
  if (comb_nsplit) HIPCHK(hipMemcpy(comb_nsplit, c->lane[0].pk.comb_nsplit, M * 4, hipMemcpyDeviceToHost));
  if (comb_tok) HIPCHK(hipMemcpy(comb_tok, c->lane[0].pk.comb_tok, M * 4, hipMemcpyDeviceToHost));
  if (units) HIPCHK(hipMemcpy(units, c->lane[0].pk.units, (size_t)c->last_units * sizeof(ifrk::AttnUnit), hipMemcpyDeviceToHost));
  if (n_units) *n_units = c->last_units;
  if (split) *split = c->last_split;
  return IFR_OK;
}

}  // extern "C"
