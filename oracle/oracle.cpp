// CPU ORACLE -- test infrastructure only.
//
// A CPU restatement of the reference's mixed-batch M-row forward.  Only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
// this library, and only as the checker or the timed CPU baseline; the
// product (intfer_amd/) never links or calls it.
//
// Each function cites the reference file:line it restates (paths relative to
// the reference root).  Two forward modes:
//   mode 0 "a8"  : the device contract -- per-token int8 activations, int32
//                  T/S accumulation, the fp32 fold, fp16 GEMM outputs, fp16 KV
//                  (or int8 KV), INT8 per-row lm_head.  Greedy tokens and
//                  logits of the HIP engine are compared against this.
//   mode 1 "f32" : the reference CpuBackend path (main.cpp:749-790): weights
//                  dequantized once to fp32, scalar row dot, fp32 KV, fp32
//                  tied-embedding lm_head (main.cpp:8302-8307).  Timed as the
//                  CPU baseline.
// Pinning of each function (what checks it beyond its own restatement) is
// listed in the header of tests/test_oracle.py.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "intfer_amd.h"

namespace {

// ---- IEEE binary16 (dashq.cpp:338-384, round-to-nearest-even) ------------
uint16_t f2h(float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t mant = x & 0x7FFFFFu;
  if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t hbit = 1u << (shift - 1);
    if (rem > hbit || (rem == hbit && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(sign | half);
}

float h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
  uint32_t mant = (uint32_t)(h & 0x3FFu);
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign << 31;
    } else {
      int e = 0;
      while (!(mant & 0x400u)) { mant <<= 1; ++e; }
      mant &= 0x3FFu;
      x = (sign << 31) | ((uint32_t)(127 - 14 - e) << 23) | (mant << 13);
    }
  } else if (exp == 0x1Fu) {
    x = (sign << 31) | 0x7F800000u | (mant << 13);
  } else {
    x = (sign << 31) | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

inline float fp16r(float v) { return h2f(f2h(v)); }

bool is_pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }
int floor_pow2(int n) { int p = 1; while (p * 2 <= n) p *= 2; return p; }

// ---- FWHT rotation (spinquant.cpp:303-312 fwht, :586-604 apply_rotation_fwht)
void fwht(float* x, int n) {
  for (int len = 2; len <= n; len <<= 1) {
    int half = len >> 1;
    for (int i = 0; i < n; i += len)
      for (int j = 0; j < half; ++j) {
        float u = x[i + j], v = x[i + j + half];
        x[i + j] = u + v;
        x[i + j + half] = u - v;
      }
  }
}

void rot(const float* x, float* out, int dim) {
  if (is_pow2(dim)) {
    for (int i = 0; i < dim; ++i) out[i] = x[i];
    fwht(out, dim);
    const float inv = 1.0f / std::sqrt((float)dim);
    for (int i = 0; i < dim; ++i) out[i] *= inv;
  } else {
    const int p = floor_pow2(dim);
    std::vector<float> tmp(x, x + p);
    fwht(tmp.data(), p);
    const float inv = 1.0f / std::sqrt((float)p);
    for (int i = 0; i < p; ++i) out[i] = tmp[i] * inv;
    for (int i = p; i < dim; ++i) out[i] = x[i];
  }
}

// ---- RMSNorm (1+w), the reference's AVX2/FMA order (main.cpp:306-351):
// eight fused lane accumulators, (lo+hi), then two horizontal adds.
void rmsnorm(const float* x, const float* w, float* out, int dim, float eps) {
  float v;
  if (dim >= 32) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= dim; i += 8)
      for (int j = 0; j < 8; ++j) acc[j] = std::fmaf(x[i + j], x[i + j], acc[j]);
    float s[4];
    for (int j = 0; j < 4; ++j) s[j] = acc[j] + acc[j + 4];
    const float h0 = s[0] + s[1], h1 = s[2] + s[3];
    v = h0 + h1;
    for (; i < dim; ++i) v += x[i] * x[i];
  } else {
    v = 0;
    for (int i = 0; i < dim; ++i) v += x[i] * x[i];
  }
  v = 1.0f / std::sqrt(v / (float)dim + eps);
  for (int i = 0; i < dim; ++i) out[i] = (x[i] * v) * (1.0f + w[i]);
}

// ---- act-quant (dashq.cpp:221-336): s = max(1e-6, max|x|)/127, inv = 1/s
// (correctly rounded), v = clamp(x*inv, +-127); HalfAway is the AVX2 form
// trunc(v + copysign(0.5, v)) (dashq.cpp:243-246), RoundNear is rint (lrint).
void act_quant_slice(const float* x, int n, int round, int8_t* q, float* scale) {
  float mx = 1e-6f;
  for (int k = 0; k < n; ++k) {
    float a = x[k] >= 0 ? x[k] : -x[k];
    if (a > mx) mx = a;
  }
  const float s = mx / 127.0f;
  const float inv = 1.0f / s;
  *scale = s;
  for (int k = 0; k < n; ++k) {
    float v = x[k] * inv;
    v = std::min(std::max(v, -127.0f), 127.0f);
    int qi;
    if (round == 0) qi = (int)std::trunc(v + std::copysign(0.5f, v));
    else qi = (int)std::nearbyint(v);
    q[k] = (int8_t)qi;
  }
}

// ---- code access (dashq.cpp:387-402 unpack_code, row-major) ---------------
inline int code_at(const ifr_linear& w, size_t n, size_t k) {
  const size_t i = n * (size_t)w.K + k;
  if (w.bits == 8) return w.codes[i];
  if (w.bits == 4) return (w.codes[i / 2] >> ((i % 2) * 4)) & 0xF;
  return (w.codes[i / 4] >> ((i % 4) * 2)) & 0x3;
}

// Per-row codes of a linear unpacked to bytes (oracle-internal cache).
struct Unpacked {
  int N = 0, K = 0, G = 0;
  std::vector<uint8_t> c;       // [N][K]
  std::vector<float> s, z;      // [N][K/G]
  float post = 1.0f;            // per-linear output factor (0 in ifr_linear reads as 1)
};

void unpack(const ifr_linear& w, Unpacked& u) {
  u.N = w.N; u.K = w.K; u.G = w.group;
  u.c.resize((size_t)w.N * w.K);
#pragma omp parallel for schedule(static)
  for (long n = 0; n < w.N; ++n)
    for (int k = 0; k < w.K; ++k) u.c[(size_t)n * w.K + k] = (uint8_t)code_at(w, n, k);
  const size_t ng = (size_t)w.N * (w.K / w.group);
  u.s.resize(ng); u.z.resize(ng);
  for (size_t i = 0; i < ng; ++i) { u.s[i] = h2f(w.scale[i]); u.z[i] = h2f(w.zero[i]); }
  u.post = w.post == 0.0f ? 1.0f : w.post;
}

// ---- quant GEMM contract (the W2A8 integer contract of dpas48_tiled,
// quant_gemm.cpp:3602-3736, with per-(row,group) scale + zero):
//   T = sum a_q*c (int32), S = sum a_q, d = fma(-z, S, T), acc = fma(s, d, acc)
//   over groups ascending; y = fp16((as * post) * acc).
void qgemm_rows(const int8_t* a, const float* as, int M, const Unpacked& u, float* y /*[M][N]*/,
                int32_t* tdump) {
  const int N = u.N, K = u.K, G = u.G, ng = K / G;
#pragma omp parallel for schedule(static) if ((long)M * N >= 2048)
  for (long r = 0; r < (long)M * N; ++r) {
    const int m = (int)(r / N), n = (int)(r % N);
    const int8_t* ar = a + (size_t)m * K;
    const uint8_t* cr = u.c.data() + (size_t)n * K;
    float acc = 0.0f;
    for (int g = 0; g < ng; ++g) {
      int32_t T = 0, S = 0;
      for (int k = g * G; k < (g + 1) * G; ++k) { T += (int32_t)ar[k] * (int32_t)cr[k]; S += ar[k]; }
      if (tdump) tdump[((size_t)m * N + n) * ng + g] = T;
      const float d = std::fmaf(-u.z[(size_t)n * ng + g], (float)S, (float)T);
      acc = std::fmaf(u.s[(size_t)n * ng + g], d, acc);
    }
    y[r] = fp16r((as[m] * u.post) * acc);
  }
}

// ---- reference CpuBackend GEMM (main.cpp:771-783): scalar dot per row.
void gemm_f32(const float* W, const float* X, float* Y, int M, int N, int K) {
#pragma omp parallel for schedule(static) if ((long)M * N >= 2048)
  for (long r = 0; r < (long)M * N; ++r) {
    const int m = (int)(r / N), i = (int)(r % N);
    const float* wr = W + (size_t)i * K;
    const float* xr = X + (size_t)m * K;
    float s = 0;
    for (int k = 0; k < K; ++k) s += wr[k] * xr[k];
    Y[r] = s;
  }
}

void dequant(const Unpacked& u, std::vector<float>& out) {
  out.resize((size_t)u.N * u.K);
  const int ng = u.K / u.G;
#pragma omp parallel for schedule(static)
  for (long n = 0; n < u.N; ++n)
    for (int k = 0; k < u.K; ++k) {
      const size_t gi = (size_t)n * ng + k / u.G;
      out[(size_t)n * u.K + k] = u.post * (u.s[gi] * ((float)u.c[(size_t)n * u.K + k] - u.z[gi]));
    }
}

// ---- lm_head INT8 per-row weights (main.cpp:1745-1761) ---------------------
void lmhead_quant(const float* W, int V, int H, int8_t* q, uint16_t* sc) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < V; ++r) {
    const float* Wr = W + (size_t)r * H;
    float mx = 0;
    for (int k = 0; k < H; ++k) { float a = std::fabs(Wr[k]); if (a > mx) mx = a; }
    const float s = (mx > 0) ? mx / 127.0f : 1.0f;
    sc[r] = f2h(s);
    const float inv = 1.0f / s;
    for (int k = 0; k < H; ++k) q[(size_t)r * H + k] = (int8_t)std::lrint(Wr[k] * inv);
  }
}

// logits(m,v) = (fold over 64-slices g: acc = fma((float)T_g, as(m,g), acc)) * ws(v)
void lmhead_rows(const int8_t* aq, const float* as, int M, const int8_t* wq, const uint16_t* ws,
                 int V, int H, float* logits) {
  const int ng = H / 64;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)M * V; ++r) {
    const int m = (int)(r / V), v = (int)(r % V);
    const int8_t* ar = aq + (size_t)m * H;
    const int8_t* wr = wq + (size_t)v * H;
    float acc = 0.0f;
    for (int g = 0; g < ng; ++g) {
      int32_t T = 0;
      for (int k = g * 64; k < g * 64 + 64; ++k) T += (int32_t)ar[k] * (int32_t)wr[k];
      acc = std::fmaf((float)T, as[(size_t)m * ng + g], acc);
    }
    logits[r] = acc * h2f(ws[v]);
  }
}

// argmax, first max wins, strict > from -1e30 (main.cpp:8289-8312)
int argmax_first(const float* x, int n) {
  int best = -1;
  float bv = -1e30f;
  for (int i = 0; i < n; ++i)
    if (x[i] > bv) { bv = x[i]; best = i; }
  return best;
}

inline float silu(float x) { return x / (1.0f + std::exp(-x)); }  // main.cpp:293

// ---- forward engine -------------------------------------------------------
struct Seq {
  bool open = false;
  int len = 0;
  std::vector<std::vector<float>> k, v;  // per layer: [len][nkv*hd] (values as stored)
};

struct Engine {
  const ifr_host_model* m = nullptr;
  ifr_model_cfg c;
  int mode = 0;     // 0 a8, 1 f32
  int kv_int8 = 0;
  // attention evaluation order: 0 the reference host loop (main.cpp:
  // 7657-7701); > 0 the split decomposition with this many KV tokens per
  // split (attn_row_split), a second faithful fp32 order of the same sum
  int attn_split = 0;
  std::vector<Unpacked> lin;           // 7 per layer (a8)
  std::vector<std::vector<float>> wf;  // 7 per layer (f32)
  std::vector<int8_t> lm_q;
  std::vector<uint16_t> lm_s;
  std::vector<float> inv_freq;
  std::vector<Seq> seqs;
};

const ifr_linear& lin_of(const ifr_layer_w& L, int j) {
  const ifr_linear* p[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
  return *p[j];
}

// rotate-half RoPE on the first rotary_dim dims (main.cpp:365-373)
void rope(const Engine& e, float* h, int pos) {
  const int half = e.c.rotary_dim / 2;
  for (int d = 0; d < half; ++d) {
    const float f = e.inv_freq[d] * (float)pos;
    const float c = std::cos(f), s = std::sin(f);
    const float a = h[d], b = h[d + half];
    h[d] = a * c - b * s;
    h[d + half] = a * s + b * c;
  }
}

// int8 KV: per (token, kv_head): s = fp16(max|x|/127) (1 if zero), q =
// half-away(x / s) clamped to +-127; stored value = q * s.
void kv_int8_round(float* x, int hd) {
  float mx = 0;
  for (int d = 0; d < hd; ++d) mx = std::max(mx, std::fabs(x[d]));
  const float s = h2f(f2h(mx > 0 ? mx / 127.0f : 1.0f));
  const float inv = 1.0f / s;
  for (int d = 0; d < hd; ++d) {
    float v = x[d] * inv;
    int q = (int)(v >= 0 ? v + 0.5f : v - 0.5f);
    q = std::min(127, std::max(-127, q));
    x[d] = (float)q * s;
  }
}

// Attention of one row in a second fp32 evaluation order, the decomposition
// the device runs: the keys [0, pos] in splits of `split` tokens; inside a
// split, pages of 32 tokens with a running (max, sum, O) in the base-2
// domain -- scores x = (q . k) * log2(e)/sqrt(hd), alpha = 2^(m_old - m_new)
// rescales sum and O when the max moves, p = 2^(x - m); then the splits are
// merged in ascending order against the largest split max, O / L.  The same
// real number as the reference loop (main.cpp:7657-7701), summed in another
// order: the spread between the two orders is the floor of what any fp32
// attention can promise.  k, v: token-major rows of nkv * hd.
void attn_row_split(const float* q, const float* k, const float* v, int pos, int nq, int nkv, int hd,
                    int split, float* out) {
  const int G = nq / nkv, kvN = nkv * hd, nt = pos + 1, ns = (nt + split - 1) / split;
  const float sl2 = 1.4426950408889634f / std::sqrt((float)hd);
  std::vector<float> ms(ns), ls(ns), os((size_t)ns * hd), x(32);
  for (int h = 0; h < nq; ++h) {
    const int kvh = h / G;
    const float* qh = q + (size_t)h * hd;
    for (int s = 0; s < ns; ++s) {
      const int lo = s * split, hi = std::min(nt, lo + split);
      float m_run = -INFINITY, l_run = 0.0f;
      float* o = &os[(size_t)s * hd];
      for (int d = 0; d < hd; ++d) o[d] = 0.0f;
      for (int p0 = lo; p0 < hi; p0 += 32) {
        const int pe = std::min(hi, p0 + 32);
        float mt = -INFINITY;
        for (int t = p0; t < pe; ++t) {
          const float* kt = k + (size_t)t * kvN + kvh * hd;
          float dot = 0.0f;
          for (int d = 0; d < hd; ++d) dot = std::fma(qh[d], kt[d], dot);
          x[t - p0] = dot * sl2;
          mt = std::max(mt, x[t - p0]);
        }
        const float m_new = std::max(m_run, mt);
        const float alpha = std::exp2(m_run - m_new);
        float rs = 0.0f;
        for (int t = p0; t < pe; ++t) {
          x[t - p0] = std::exp2(x[t - p0] - m_new);
          rs += x[t - p0];
        }
        l_run = l_run * alpha + rs;
        if (alpha != 1.0f)
          for (int d = 0; d < hd; ++d) o[d] *= alpha;
        for (int t = p0; t < pe; ++t) {
          const float* vt = v + (size_t)t * kvN + kvh * hd;
          for (int d = 0; d < hd; ++d) o[d] = std::fma(x[t - p0], vt[d], o[d]);
        }
        m_run = m_new;
      }
      ms[s] = m_run;
      ls[s] = l_run;
    }
    float mx = -INFINITY;
    for (int s = 0; s < ns; ++s) mx = std::max(mx, ms[s]);
    float L = 0.0f;
    float* oh = out + (size_t)h * hd;
    for (int d = 0; d < hd; ++d) oh[d] = 0.0f;
    for (int s = 0; s < ns; ++s) {
      const float f = std::exp2(ms[s] - mx);
      L += f * ls[s];
      for (int d = 0; d < hd; ++d) oh[d] += f * os[(size_t)s * hd + d];
    }
    const float invL = 1.0f / L;
    for (int d = 0; d < hd; ++d) oh[d] *= invL;
  }
}

// One linear over M rows.  a8: x is quantized per token (half-away) here.
void linear(Engine& e, int layer, int j, const float* x, int M, float* y) {
  const ifr_linear& w = lin_of(e.m->layers[layer], j);
  if (e.mode == 1) {
    gemm_f32(e.wf[(size_t)layer * 7 + j].data(), x, y, M, w.N, w.K);
    return;
  }
  std::vector<int8_t> q((size_t)M * w.K);
  std::vector<float> as(M);
  for (int m = 0; m < M; ++m)
    act_quant_slice(x + (size_t)m * w.K, w.K, 0, q.data() + (size_t)m * w.K, &as[m]);
  qgemm_rows(q.data(), as.data(), M, e.lin[(size_t)layer * 7 + j], y, nullptr);
}

int forward(Engine& e, const ifr_row* rows, int M, int32_t* best, float* logits_out) {
  const ifr_model_cfg& c = e.c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv, F = c.inter;
  const int qN = nq * hd, kvN = nkv * hd, Gq = nq / nkv;
  // Validate rows: per sequence contiguous, positions consecutive from len.
  for (int m = 0; m < M; ++m) {
    const ifr_row& r = rows[m];
    if (r.seq < 0 || r.seq >= (int)e.seqs.size() || !e.seqs[r.seq].open) return IFR_EINVAL;
    if (r.token < 0 || r.token >= c.vocab) return IFR_EINVAL;
    const bool first = (m == 0 || rows[m - 1].seq != r.seq);
    if (first) {
      if (r.pos != e.seqs[r.seq].len) return IFR_EINVAL;
      for (int p = 0; p < m; ++p) if (rows[p].seq == r.seq) return IFR_EINVAL;
    } else if (r.pos != rows[m - 1].pos + 1) {
      return IFR_EINVAL;
    }
  }
  std::vector<float> Hs((size_t)M * H);
  for (int m = 0; m < M; ++m)  // embedding gather (main.cpp:7531-7537)
    std::memcpy(&Hs[(size_t)m * H], e.m->embed + (size_t)rows[m].token * H, H * sizeof(float));
  std::vector<float> normed((size_t)M * H), rin((size_t)M * H), qkv((size_t)M * (qN + 2 * kvN));
  std::vector<float> qb((size_t)M * qN), kb((size_t)M * kvN), vb((size_t)M * kvN);
  // gated q_proj output [M][2 qN] (per head: q rows, then gate rows) and the gate
  std::vector<float> qg(c.attn_gate ? (size_t)M * 2 * qN : 0), gate(c.attn_gate ? (size_t)M * qN : 0);
  std::vector<float> attn((size_t)M * qN), y((size_t)M * H), tmp(H);
  std::vector<float> g((size_t)M * F), u((size_t)M * F);
  // grow KV
  for (int m = 0; m < M; ++m) {
    Seq& s = e.seqs[rows[m].seq];
    for (int l = 0; l < c.layers; ++l) {
      s.k[l].resize((size_t)(rows[m].pos + 1) * kvN);
      s.v[l].resize((size_t)(rows[m].pos + 1) * kvN);
    }
  }
  for (int l = 0; l < c.layers; ++l) {
    const ifr_layer_w& Lw = e.m->layers[l];
    for (int m = 0; m < M; ++m) {
      rmsnorm(&Hs[(size_t)m * H], Lw.in_ln, &normed[(size_t)m * H], H, c.rms_eps);
      if (c.rotate) rot(&normed[(size_t)m * H], &rin[(size_t)m * H], H);
      else std::memcpy(&rin[(size_t)m * H], &normed[(size_t)m * H], H * sizeof(float));
    }
    if (c.attn_gate) {
      // [q, gate] interleaved per head (main.cpp:7625-7640)
      linear(e, l, 0, rin.data(), M, qg.data());
      for (int m = 0; m < M; ++m)
        for (int h = 0; h < nq; ++h)
          for (int d = 0; d < hd; ++d) {
            qb[(size_t)m * qN + h * hd + d] = qg[(size_t)m * 2 * qN + 2 * h * hd + d];
            gate[(size_t)m * qN + h * hd + d] = qg[(size_t)m * 2 * qN + 2 * h * hd + hd + d];
          }
    } else {
      linear(e, l, 0, rin.data(), M, qb.data());
    }
    linear(e, l, 1, rin.data(), M, kb.data());
    linear(e, l, 2, rin.data(), M, vb.data());
    // q/k norm, RoPE, KV append: all rows first (main.cpp:7625-7656)
    for (int m = 0; m < M; ++m) {
      const int pos = rows[m].pos;
      float* qr = &qb[(size_t)m * qN];
      float* kr = &kb[(size_t)m * kvN];
      float* vr = &vb[(size_t)m * kvN];
      for (int h = 0; h < nq; ++h) {
        if (c.qk_norm) rmsnorm(qr + h * hd, Lw.q_norm, qr + h * hd, hd, c.rms_eps);
        rope(e, qr + h * hd, pos);
      }
      for (int h = 0; h < nkv; ++h) {
        if (c.qk_norm) rmsnorm(kr + h * hd, Lw.k_norm, kr + h * hd, hd, c.rms_eps);
        rope(e, kr + h * hd, pos);
      }
      if (e.mode == 0) {
        for (int i = 0; i < qN; ++i) qr[i] = fp16r(qr[i]);
        for (int i = 0; i < kvN; ++i) { kr[i] = fp16r(kr[i]); vr[i] = fp16r(vr[i]); }
        if (e.kv_int8)
          for (int h = 0; h < nkv; ++h) { kv_int8_round(kr + h * hd, hd); kv_int8_round(vr + h * hd, hd); }
      }
      Seq& s = e.seqs[rows[m].seq];
      std::memcpy(&s.k[l][(size_t)pos * kvN], kr, kvN * sizeof(float));
      std::memcpy(&s.v[l][(size_t)pos * kvN], vr, kvN * sizeof(float));
    }
    // host attention, reference loop order (main.cpp:7657-7701), or the
    // split order (attn_row_split)
#pragma omp parallel for schedule(dynamic) if (e.mode == 0)
    for (int m = 0; m < M; ++m) {
      const int pos = rows[m].pos;
      const Seq& s = e.seqs[rows[m].seq];
      if (e.attn_split > 0) {
        attn_row_split(&qb[(size_t)m * qN], s.k[l].data(), s.v[l].data(), pos, nq, nkv, hd, e.attn_split,
                       &attn[(size_t)m * qN]);
        if (c.attn_gate && !c.attn_gate_off)
          for (int i = 0; i < qN; ++i)
            attn[(size_t)m * qN + i] *= 1.0f / (1.0f + std::exp(-gate[(size_t)m * qN + i]));
        continue;
      }
      std::vector<float> gs((size_t)Gq * (pos + 1));
      float* at = &attn[(size_t)m * qN];
      const float* qr = &qb[(size_t)m * qN];
      for (int kvh = 0; kvh < nkv; ++kvh) {
        float mx[64];
        for (int j = 0; j < Gq; ++j) mx[j] = -1e30f;
        for (int t = 0; t <= pos; ++t) {
          const float* kh = &s.k[l][(size_t)t * kvN + kvh * hd];
          for (int j = 0; j < Gq; ++j) {
            const float* qh = qr + (kvh * Gq + j) * hd;
            float sc = 0;
            for (int d = 0; d < hd; ++d) sc += qh[d] * kh[d];
            sc *= 1.0f / std::sqrt((float)hd);
            gs[(size_t)j * (pos + 1) + t] = sc;
            if (sc > mx[j]) mx[j] = sc;
          }
        }
        for (int j = 0; j < Gq; ++j) {
          float* row = &gs[(size_t)j * (pos + 1)];
          float sum = 0;
          for (int t = 0; t <= pos; ++t) { row[t] = std::exp(row[t] - mx[j]); sum += row[t]; }
          for (int t = 0; t <= pos; ++t) row[t] /= sum;
        }
        for (int j = 0; j < Gq; ++j) {
          float* oh = at + (kvh * Gq + j) * hd;
          for (int d = 0; d < hd; ++d) oh[d] = 0;
        }
        for (int t = 0; t <= pos; ++t) {
          const float* vh = &s.v[l][(size_t)t * kvN + kvh * hd];
          for (int j = 0; j < Gq; ++j) {
            const float st = gs[(size_t)j * (pos + 1) + t];
            float* oh = at + (kvh * Gq + j) * hd;
            for (int d = 0; d < hd; ++d) oh[d] += st * vh[d];
          }
        }
      }
      // output gate (main.cpp:7697-7698; sigmoidf of main.cpp:294)
      if (c.attn_gate && !c.attn_gate_off)
        for (int i = 0; i < qN; ++i) at[i] *= 1.0f / (1.0f + std::exp(-gate[(size_t)m * qN + i]));
    }
    // o-proj, rot_left, residual (main.cpp:7702-7727)
    linear(e, l, 3, attn.data(), M, y.data());
    for (int m = 0; m < M; ++m) {
      float* hr = &Hs[(size_t)m * H];
      const float* yr = &y[(size_t)m * H];
      if (c.rotate) rot(yr, tmp.data(), H); else std::memcpy(tmp.data(), yr, H * sizeof(float));
      for (int i = 0; i < H; ++i) hr[i] += tmp[i];
      rmsnorm(hr, Lw.post_ln, &normed[(size_t)m * H], H, c.rms_eps);
      if (c.rotate) rot(&normed[(size_t)m * H], &rin[(size_t)m * H], H);
      else std::memcpy(&rin[(size_t)m * H], &normed[(size_t)m * H], H * sizeof(float));
    }
    // MLP (main.cpp:7740-7772)
    linear(e, l, 4, rin.data(), M, g.data());
    linear(e, l, 5, rin.data(), M, u.data());
    for (size_t i = 0; i < g.size(); ++i) {
      const float v = silu(g[i]) * u[i];
      g[i] = (e.mode == 0) ? fp16r(v) : v;
    }
    linear(e, l, 6, g.data(), M, y.data());
    for (int m = 0; m < M; ++m) {
      float* hr = &Hs[(size_t)m * H];
      const float* yr = &y[(size_t)m * H];
      if (c.rotate) rot(yr, tmp.data(), H); else std::memcpy(tmp.data(), yr, H * sizeof(float));
      for (int i = 0; i < H; ++i) hr[i] += tmp[i];
    }
  }
  for (int m = 0; m < M; ++m) e.seqs[rows[m].seq].len = rows[m].pos + 1;
  // final norm + lm_head + argmax (main.cpp:8231-8317)
  // The reference scores every row (main.cpp:8231-8232); the f32 mode keeps
  // that cost and reports the requested rows.  The a8 mode scores requested
  // rows only, like the device.
  std::vector<int> want, report;
  for (int m = 0; m < M; ++m) {
    best[m] = -1;
    if (rows[m].want || e.mode == 1) want.push_back(m);
    if (rows[m].want) report.push_back(m);
  }
  const int W = (int)want.size();
  if (W == 0) return IFR_OK;
  std::vector<float> fn((size_t)W * H), lg((size_t)W * c.vocab);
  for (int i = 0; i < W; ++i)
    rmsnorm(&Hs[(size_t)want[i] * H], e.m->final_norm, &fn[(size_t)i * H], H, c.rms_eps);
  if (e.mode == 0) {
    const int ng = H / 64;
    std::vector<int8_t> aq((size_t)W * H);
    std::vector<float> as((size_t)W * ng);
    for (int i = 0; i < W; ++i)
      for (int gg = 0; gg < ng; ++gg)
        act_quant_slice(&fn[(size_t)i * H + gg * 64], 64, 1, &aq[(size_t)i * H + gg * 64],
                        &as[(size_t)i * ng + gg]);
    lmhead_rows(aq.data(), as.data(), W, e.lm_q.data(), e.lm_s.data(), c.vocab, H, lg.data());
  } else {
    // fp32 lm_head (the tied embedding unless the model has its own),
    // serial as in the reference (main.cpp:8302-8307)
    const float* lmw = e.m->lm_head ? e.m->lm_head : e.m->embed;
    for (int i = 0; i < W; ++i)
      for (int v = 0; v < c.vocab; ++v) {
        const float* er = lmw + (size_t)v * H;
        const float* f = &fn[(size_t)i * H];
        float s = 0;
        for (int k = 0; k < H; ++k) s += f[k] * er[k];
        lg[(size_t)i * c.vocab + v] = s;
      }
  }
  int out_i = 0;
  for (int i = 0; i < W; ++i) {
    if (!rows[want[i]].want) continue;
    best[want[i]] = argmax_first(&lg[(size_t)i * c.vocab], c.vocab);
    if (logits_out)
      std::memcpy(logits_out + (size_t)out_i * c.vocab, &lg[(size_t)i * c.vocab], c.vocab * sizeof(float));
    ++out_i;
  }
  (void)report;
  return IFR_OK;
}

}  // namespace

extern "C" {

uint16_t or_f2h(float v) { return f2h(v); }
float or_h2f(uint16_t h) { return h2f(h); }
void or_f2h_batch(const float* x, uint16_t* y, size_t n) { for (size_t i = 0; i < n; ++i) y[i] = f2h(x[i]); }
void or_h2f_batch(const uint16_t* x, float* y, size_t n) { for (size_t i = 0; i < n; ++i) y[i] = h2f(x[i]); }

void or_rot(const float* x, float* out, int dim) { rot(x, out, dim); }
void or_fwht(float* x, int n) { fwht(x, n); }

void or_rmsnorm(const float* x, const float* w, float* out, int dim, float eps) {
  rmsnorm(x, w, out, dim, eps);
}

// Per row of K: optional RMSNorm(1+w), optional rotation, then act-quant in
// slices of ga (0 = whole row).  gsum (may be NULL) gets the per-128-group
// sum of the codes as float.
void or_act_quant(const float* x, int M, int K, const float* norm_w, float eps, int rotate,
                  int round, int ga, int8_t* q, float* scales, float* gsum) {
  const int sl = ga > 0 ? ga : K;
  const int ns = K / sl;
  std::vector<float> a(K), b(K);
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (size_t)m * K;
    if (norm_w) { rmsnorm(xr, norm_w, a.data(), K, eps); xr = a.data(); }
    if (rotate) { rot(xr, b.data(), K); xr = b.data(); }
    for (int s = 0; s < ns; ++s)
      act_quant_slice(xr + s * sl, sl, round, q + (size_t)m * K + s * sl, scales + (size_t)m * ns + s);
    if (gsum)
      for (int g = 0; g < K / 128; ++g) {
        int32_t S = 0;
        for (int k = g * 128; k < g * 128 + 128; ++k) S += q[(size_t)m * K + k];
        gsum[(size_t)m * (K / 128) + g] = (float)S;
      }
  }
}

// Brute-force integer T(m,n,g) and S(m,g) (int32).
void or_qgemm_ts(const int8_t* a, int M, const ifr_linear* w, int32_t* T, int32_t* S) {
  const int N = w->N, K = w->K, G = w->group, ng = K / G;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)M * N; ++r) {
    const int m = (int)(r / N), n = (int)(r % N);
    for (int g = 0; g < ng; ++g) {
      int32_t t = 0;
      for (int k = g * G; k < (g + 1) * G; ++k) t += (int32_t)a[(size_t)m * K + k] * code_at(*w, n, k);
      T[((size_t)m * N + n) * ng + g] = t;
    }
  }
  if (S)
    for (int m = 0; m < M; ++m)
      for (int g = 0; g < ng; ++g) {
        int32_t s = 0;
        for (int k = g * G; k < (g + 1) * G; ++k) s += a[(size_t)m * K + k];
        S[(size_t)m * ng + g] = s;
      }
}

// The quant GEMM contract, fp16 output bits.
void or_qgemm(const int8_t* a, const float* as, int M, const ifr_linear* w, uint16_t* out) {
  Unpacked u;
  unpack(*w, u);
  std::vector<float> y((size_t)M * w->N);
  qgemm_rows(a, as, M, u, y.data(), nullptr);
  for (size_t i = 0; i < y.size(); ++i) out[i] = f2h(y[i]);
}

// The reference's DPAS fold with grouped activation scales (dpas48_tiled,
// src/gemm/quant_gemm.cpp:3492-3791; the per-op math :3602-3736, act_group
// GA :3502, As[r][k0 / GA] :3614).  For each 32-wide K op o in ascending
// order (k0 = 32 o): T = sum a_q c and S = sum a_q over the op (exact int32,
// c the code 0..C), and
//     acc += as[m][k0 / GA] * ws[n][k0 / G] * alpha * (2T - C S) * (1 / C)
// evaluated in the source's left-to-right order in fp32, every product and
// the add rounded (no contraction); out = fp16_rne(acc) (to_half_bits :84).
// 2T - C S is an integer below 2^24, exact in fp32 however it is formed.
// a: int8 [M][K] row-major, as: fp32 [M][K / GA].
void or_qgemm_ga(const int8_t* a, const float* as, int M, int ga, const ifr_linear* w, float alpha,
                 uint16_t* out) {
  Unpacked u;
  unpack(*w, u);
  const int N = u.N, K = u.K, G = u.G;
  const float C = (float)((1 << w->bits) - 1);
  const float Cinv = 1.0f / C;
#pragma omp parallel for schedule(static) if ((long)M * N >= 2048)
  for (long r = 0; r < (long)M * N; ++r) {
    const int m = (int)(r / N), n = (int)(r % N);
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 32) {
      int32_t T = 0, S = 0;
      for (int k = k0; k < k0 + 32; ++k) {
        const int32_t av = a[(size_t)m * K + k];
        T += av * (int32_t)u.c[(size_t)n * K + k];
        S += av;
      }
      const float asv = as[(size_t)m * (K / ga) + k0 / ga];
      const float ws = u.s[(size_t)n * (K / G) + k0 / G];
      const float d = 2.0f * (float)T - C * (float)S;
      float x = asv * ws;
      x = x * alpha;
      x = x * d;
      x = x * Cinv;
      acc = acc + x;
    }
    out[r] = f2h(acc);
  }
}

// SwiGLU over two fp16 GEMM outputs: fp16(silu(g) * u).
void or_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f2h(silu(h2f(g[i])) * h2f(u[i]));
}

// FP16-activation dequant GEMM (quant_gemm_forward_usm,
// src/gemm/quant_gemm.cpp:359-2153): w(n,k) = (half(scale) * alpha) *
// canon_value(bits, code) (:139-144, fp32), out = fp16(sum_k a * w) with an
// fp32 accumulator in ascending k.  M == 1 (decode1 kernels :1026-1080,
// :2022-2066): w in fp32 and `acc += av * w` taken as one fused
// multiply-add; M > 1 (tiled kernel :2069-2150): w rounded to fp16 as staged,
// so a * w is exact and the step is one rounded add.
void or_qgemm_f16(const uint16_t* a, int M, const ifr_linear* w, float alpha, uint16_t* out) {
  Unpacked u;
  unpack(*w, u);
  const int N = u.N, K = u.K, G = u.G, bits = w->bits;
  const float Cf = (float)((1 << bits) - 1);
  auto canon = [&](int c) -> float {
    if (bits >= 8) return (2.0f * (float)c - 255.0f) / 255.0f;
    if (bits == 4) return (2.0f * (float)c - 15.0f) / 15.0f;
    static const float c2[4] = {-1.0f, -1.0f / 3.0f, 1.0f / 3.0f, 1.0f};
    return c2[c & 3];
  };
  (void)Cf;
#pragma omp parallel for schedule(static) if ((long)M * N >= 2048)
  for (long r = 0; r < (long)M * N; ++r) {
    const int m = (int)(r / N), n = (int)(r % N);
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
      const float s = u.s[(size_t)n * (K / G) + k / G] * alpha;
      float wv = s * canon(u.c[(size_t)n * K + k]);
      if (M > 1) wv = h2f(f2h(wv));
      acc = std::fmaf(h2f(a[(size_t)m * K + k]), wv, acc);
    }
    out[r] = f2h(acc);
  }
}

void or_dequant(const ifr_linear* w, float* out) {
  Unpacked u;
  unpack(*w, u);
  std::vector<float> d;
  dequant(u, d);
  std::memcpy(out, d.data(), d.size() * sizeof(float));
}

void or_gemm_f32(const float* W, const float* X, float* Y, int M, int N, int K) {
  gemm_f32(W, X, Y, M, N, K);
}

void or_lmhead_quant(const float* W, int V, int H, int8_t* q, uint16_t* sc) {
  lmhead_quant(W, V, H, q, sc);
}

void or_lmhead(const int8_t* aq, const float* as, int M, const int8_t* wq, const uint16_t* ws,
               int V, int H, float* logits, int32_t* best) {
  lmhead_rows(aq, as, M, wq, ws, V, H, logits);
  if (best)
    for (int m = 0; m < M; ++m) best[m] = argmax_first(logits + (size_t)m * V, V);
}

int or_argmax(const float* x, int n) { return argmax_first(x, n); }

// RoPE on one head vector with the reference inv_freq (main.cpp:10594-10596).
void or_rope(float* h, int pos, int rotary_dim, float theta) {
  Engine e;
  e.c.rotary_dim = rotary_dim;
  e.inv_freq.resize(rotary_dim / 2);
  for (int d = 0; d < rotary_dim / 2; ++d)
    e.inv_freq[d] = 1.0f / std::pow(theta, (2.0f * d) / (float)rotary_dim);
  rope(e, h, pos);
}

// Reference host attention for one row against given K/V (fp32 values):
// q [nq*hd], k/v [(pos+1)][nkv*hd] -> out [nq*hd].
void or_attention_row(const float* q, const float* k, const float* v, int pos, int nq, int nkv,
                      int hd, float* out) {
  const int G = nq / nkv, kvN = nkv * hd;
  std::vector<float> gs((size_t)G * (pos + 1));
  for (int kvh = 0; kvh < nkv; ++kvh) {
    float mx[64];
    for (int j = 0; j < G; ++j) mx[j] = -1e30f;
    for (int t = 0; t <= pos; ++t) {
      const float* kh = k + (size_t)t * kvN + kvh * hd;
      for (int j = 0; j < G; ++j) {
        const float* qh = q + (kvh * G + j) * hd;
        float sc = 0;
        for (int d = 0; d < hd; ++d) sc += qh[d] * kh[d];
        sc *= 1.0f / std::sqrt((float)hd);
        gs[(size_t)j * (pos + 1) + t] = sc;
        if (sc > mx[j]) mx[j] = sc;
      }
    }
    for (int j = 0; j < G; ++j) {
      float* row = &gs[(size_t)j * (pos + 1)];
      float sum = 0;
      for (int t = 0; t <= pos; ++t) { row[t] = std::exp(row[t] - mx[j]); sum += row[t]; }
      for (int t = 0; t <= pos; ++t) row[t] /= sum;
      float* oh = out + (kvh * G + j) * hd;
      for (int d = 0; d < hd; ++d) oh[d] = 0;
    }
    for (int t = 0; t <= pos; ++t) {
      const float* vh = v + (size_t)t * kvN + kvh * hd;
      for (int j = 0; j < G; ++j) {
        const float st = gs[(size_t)j * (pos + 1) + t];
        float* oh = out + (kvh * G + j) * hd;
        for (int d = 0; d < hd; ++d) oh[d] += st * vh[d];
      }
    }
  }
}

void or_kv_int8_round(float* x, int hd) { kv_int8_round(x, hd); }
// n consecutive vectors of hd (a whole cache at once)
void or_kv_int8_round_rows(float* x, long n, int hd) {
  for (long i = 0; i < n; ++i) kv_int8_round(x + i * hd, hd);
}
void or_attention_row_split(const float* q, const float* k, const float* v, int pos, int nq, int nkv, int hd,
                            int split, float* out) {
  attn_row_split(q, k, v, pos, nq, nkv, hd, split, out);
}
// the attention order of an engine's forward (0: reference loop; > 0: split)
int or_engine_set_attn_split(void* p, int split) {
  if (split < 0 || split % 32) return IFR_EINVAL;
  static_cast<Engine*>(p)->attn_split = split;
  return IFR_OK;
}

// ---- sampling: the reference's sample() (main.cpp:8674-8764, default path;
// the INTFER_SAMPLE_TOPK_DIRECT variant :8695-8724 is opt-in) over the
// request's std::mt19937 (main.cpp:4815, seeded :9305), with the draw taken
// by std::uniform_real_distribution<float>(0, 1) of the standard library,
// exactly as the reference takes it.
void* or_rng_create(uint32_t seed) { return new std::mt19937(seed); }
void or_rng_free(void* g) { delete static_cast<std::mt19937*>(g); }
uint32_t or_rng_next(void* g) { return (uint32_t)(*static_cast<std::mt19937*>(g))(); }
float or_rng_uniform(void* g) {
  std::uniform_real_distribution<float> U(0.f, 1.f);
  return U(*static_cast<std::mt19937*>(g));
}
int or_sample(const float* logits, int V, int top_k, float top_p, float temperature, void* g) {
  std::mt19937& rng = *static_cast<std::mt19937*>(g);
  if (temperature <= 0.f) temperature = 1e-5f;                     // :8676
  float mx = -1e30f;                                                // :8725-8726
  for (int i = 0; i < V; ++i)
    if (logits[i] > mx) mx = logits[i];
  std::vector<float> probs((size_t)V);
  float sum = 0.f;                                                  // :8730-8735
  for (int i = 0; i < V; ++i) {
    probs[(size_t)i] = expf((logits[i] - mx) / temperature);
    sum += probs[(size_t)i];
  }
  for (float& q : probs) q /= sum;                                  // :8736
  auto renorm = [&]() {
    sum = 0.f;
    for (float q : probs) sum += q;
    for (float& q : probs) q /= sum;
  };
  if (top_k > 0 && V > top_k) {                                     // :8737-8743
    std::vector<float> sorted = probs;
    std::nth_element(sorted.begin(), sorted.end() - top_k, sorted.end());
    const float kth = sorted[sorted.size() - (size_t)top_k];
    for (float& q : probs)
      if (q < kth) q = 0.f;
    renorm();
  }
  if (top_p > 0.f && top_p < 1.f) {                                 // :8744-8756
    std::vector<int> idx((size_t)V);
    for (int i = 0; i < V; ++i) idx[(size_t)i] = i;
    std::sort(idx.begin(), idx.end(), [&](int a, int b) { return probs[(size_t)a] > probs[(size_t)b]; });
    float cum = 0.f;
    int cutoff = V;
    for (int i = 0; i < V; ++i) {
      cum += probs[(size_t)idx[(size_t)i]];
      if (cum >= top_p) { cutoff = i + 1; break; }
    }
    for (int i = cutoff; i < V; ++i) probs[(size_t)idx[(size_t)i]] = 0.f;
    renorm();
  }
  std::uniform_real_distribution<float> U(0.f, 1.f);               // :8757-8763
  const float r = U(rng);
  float acc = 0.f;
  for (int i = 0; i < V; ++i) {
    acc += probs[(size_t)i];
    if (r <= acc) return i;
  }
  return V - 1;
}

void* or_engine_create(const ifr_host_model* m, int kv_int8, int mode, int max_seqs) {
  if (!m || (mode != 0 && mode != 1)) return nullptr;
  auto* e = new Engine();
  e->m = m;
  e->c = m->cfg;
  e->mode = mode;
  e->kv_int8 = kv_int8;
  const int L = e->c.layers;
  if (mode == 0) {
    e->lin.resize((size_t)L * 7);
    for (int l = 0; l < L; ++l)
      for (int j = 0; j < 7; ++j) unpack(lin_of(m->layers[l], j), e->lin[(size_t)l * 7 + j]);
    e->lm_q.resize((size_t)e->c.vocab * e->c.hidden);
    e->lm_s.resize(e->c.vocab);
    lmhead_quant(m->lm_head ? m->lm_head : m->embed, e->c.vocab, e->c.hidden, e->lm_q.data(),
                 e->lm_s.data());
  } else {
    e->wf.resize((size_t)L * 7);
    for (int l = 0; l < L; ++l)
      for (int j = 0; j < 7; ++j) {
        Unpacked u;
        unpack(lin_of(m->layers[l], j), u);
        dequant(u, e->wf[(size_t)l * 7 + j]);
      }
  }
  e->inv_freq.resize(e->c.rotary_dim / 2);
  for (int d = 0; d < e->c.rotary_dim / 2; ++d)
    e->inv_freq[d] = 1.0f / std::pow(e->c.rope_theta, (2.0f * d) / (float)e->c.rotary_dim);
  e->seqs.resize(max_seqs);
  return e;
}

void or_engine_destroy(void* p) { delete static_cast<Engine*>(p); }

int or_seq_open(void* p) {
  Engine* e = static_cast<Engine*>(p);
  for (size_t i = 0; i < e->seqs.size(); ++i)
    if (!e->seqs[i].open) {
      Seq& s = e->seqs[i];
      s.open = true;
      s.len = 0;
      s.k.assign(e->c.layers, {});
      s.v.assign(e->c.layers, {});
      return (int)i;
    }
  return -1;
}

void or_seq_close(void* p, int slot) {
  Engine* e = static_cast<Engine*>(p);
  if (slot >= 0 && slot < (int)e->seqs.size()) e->seqs[slot] = Seq();
}

int or_seq_truncate(void* p, int slot, int len) {
  Engine* e = static_cast<Engine*>(p);
  if (slot < 0 || slot >= (int)e->seqs.size() || !e->seqs[slot].open) return IFR_EINVAL;
  Seq& s = e->seqs[slot];
  if (len < 0 || len > s.len) return IFR_EINVAL;
  const size_t kvN = (size_t)e->c.n_kv * e->c.head_dim;
  for (int l = 0; l < e->c.layers; ++l) { s.k[l].resize(len * kvN); s.v[l].resize(len * kvN); }
  s.len = len;
  return IFR_OK;
}

// Pre-fill a sequence's cache with given per-layer K/V values (fp32 [len][nkv*hd]
// per layer, layer-major), e.g. seeded N(0,1) contexts of the configs.
int or_seq_set_kv(void* p, int slot, int len, const float* k, const float* v) {
  Engine* e = static_cast<Engine*>(p);
  if (slot < 0 || slot >= (int)e->seqs.size() || !e->seqs[slot].open) return IFR_EINVAL;
  Seq& s = e->seqs[slot];
  const size_t kvN = (size_t)e->c.n_kv * e->c.head_dim, per = (size_t)len * kvN;
  for (int l = 0; l < e->c.layers; ++l) {
    s.k[l].assign(k + l * per, k + (l + 1) * per);
    s.v[l].assign(v + l * per, v + (l + 1) * per);
  }
  s.len = len;
  return IFR_OK;
}

int or_forward(void* p, const ifr_row* rows, int M, int32_t* best, float* logits) {
  return forward(*static_cast<Engine*>(p), rows, M, best, logits);
}

}  // extern "C"
