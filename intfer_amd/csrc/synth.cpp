// Seeded synthetic decoder weights for the 0.8B-class and 27B-class configs.
//
// Portable by construction: splitmix64 for bits, explicit Box-Muller in double
// for normals (std::normal_distribution is implementation-defined), fixed
// 65536-element substreams so the result does not depend on the thread count.
//
// Distributions (recorded so the CPU oracle and the device see one model):
//   codes          uniform over [0, 2^bits)
//   scale(n,g)     fp16(|N(0, 0.02)|)
//   zero(n,g)      fp16((2^bits - 1) / 2)       (the reference codebook centre)
//   embed          N(0, 0.02)                    (tied with lm_head; a small
//                  embedding keeps the input token from dominating its own
//                  logit, so greedy streams are not degenerate)
//   norm weights   N(0, 0.1)   used as (1 + w)   (Qwen3.5 offset form)
// bits_mode 0 draws each linear's width with P(INT2) = 0.7, else INT4
// (a seeded stand-in for the reference's RCO budget split, src/quant/rco.cpp).
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "host_model.h"
#include "ifr_half.h"

namespace ifrh {

void OwnedModel::publish() {
  const int L = pub.cfg.layers;
  layers.resize(L);
  for (int l = 0; l < L; ++l) {
    ifr_layer_w& w = layers[l];
    w.in_ln = norms[(size_t)l * 4 + 0].data();
    w.post_ln = norms[(size_t)l * 4 + 1].data();
    w.q_norm = norms[(size_t)l * 4 + 2].empty() ? nullptr : norms[(size_t)l * 4 + 2].data();
    w.k_norm = norms[(size_t)l * 4 + 3].empty() ? nullptr : norms[(size_t)l * 4 + 3].data();
    ifr_linear* slots[7] = {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down};
    for (int j = 0; j < 7; ++j) {
      const OwnedLinear& o = lin[(size_t)l * 7 + j];
      slots[j]->codes = o.codes.data();
      slots[j]->scale = o.scale.data();
      slots[j]->zero = o.zero.data();
    }
  }
  pub.embed = embed.data();
  pub.final_norm = final_norm.data();
  pub.layers = layers.data();
  pub.lm_head = lm_head.empty() ? nullptr : lm_head.data();
}

namespace {
std::mutex g_models_mu;
std::map<ifr_host_model*, OwnedModel*> g_models;
}  // namespace

ifr_host_model* adopt(OwnedModel* m) {
  std::lock_guard<std::mutex> lk(g_models_mu);
  g_models[&m->pub] = m;
  return &m->pub;
}

}  // namespace ifrh

namespace {

using ifrh::OwnedLinear;
using ifrh::OwnedModel;

inline uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t stream_seed(uint64_t seed, uint64_t tensor, uint64_t chunk) {
  uint64_t s = seed ^ (tensor * 0xD1B54A32D192ED03ull) ^ (chunk * 0x8CB92BA72F3D8DD7ull);
  splitmix64(s);
  return splitmix64(s);
}

constexpr size_t kChunk = 65536;

// Fill out[0..n) with N(0, sigma) (Box-Muller, both outputs used).
void fill_normal(float* out, size_t n, float sigma, uint64_t seed, uint64_t tensor) {
  const size_t nchunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(static)
  for (long c = 0; c < (long)nchunks; ++c) {
    uint64_t s = stream_seed(seed, tensor, (uint64_t)c);
    const size_t i0 = (size_t)c * kChunk;
    const size_t i1 = (i0 + kChunk < n) ? i0 + kChunk : n;
    for (size_t i = i0; i < i1; i += 2) {
      const double u1 = ((double)(splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
      const double u2 = (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
      const double r = std::sqrt(-2.0 * std::log(u1));
      const double t = 6.283185307179586 * u2;
      out[i] = (float)(r * std::cos(t) * sigma);
      if (i + 1 < i1) out[i + 1] = (float)(r * std::sin(t) * sigma);
    }
  }
}

// Uniform codes, packed row-major LSB-first at `bits` per code.
void fill_codes(uint8_t* out, size_t ncodes, int bits, uint64_t seed, uint64_t tensor) {
  const size_t nbytes = ncodes * (size_t)bits / 8;
  const size_t nchunks = (nbytes + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(static)
  for (long c = 0; c < (long)nchunks; ++c) {
    uint64_t s = stream_seed(seed, tensor, (uint64_t)c);
    const size_t b0 = (size_t)c * kChunk;
    const size_t b1 = (b0 + kChunk < nbytes) ? b0 + kChunk : nbytes;
    for (size_t b = b0; b < b1; b += 8) {
      uint64_t r = splitmix64(s);
      for (size_t j = 0; j < 8 && b + j < b1; ++j) out[b + j] = (uint8_t)(r >> (8 * j));
    }
  }
}

// intfer_form: one scale per K-group shared by all rows (drawn per group),
// post = 2/C, so the linear is exactly what an .intfer file stores.
void make_linear(OwnedLinear& o, ifr_linear& L, int N, int K, int bits, int group,
                 uint64_t seed, uint64_t tid, bool intfer_form) {
  const size_t n = (size_t)N * K;
  o.codes.resize(n * (size_t)bits / 8);
  fill_codes(o.codes.data(), n, bits, seed, tid * 4 + 0);
  const size_t ngk = (size_t)(K / group), ng = (size_t)N * ngk;
  std::vector<float> sc(intfer_form ? ngk : ng);
  fill_normal(sc.data(), sc.size(), 0.02f, seed, tid * 4 + 1);
  o.scale.resize(ng);
  o.zero.resize(ng);
  const int C = (1 << bits) - 1;
  const uint16_t z = ifr::f2h((float)C * 0.5f);
  for (size_t i = 0; i < ng; ++i) {
    o.scale[i] = ifr::f2h(std::fabs(sc[intfer_form ? i % ngk : i]));
    o.zero[i] = z;
  }
  L.N = N; L.K = K; L.bits = bits; L.group = group;
  L.post = intfer_form ? 2.0f / (float)C : 0.0f;
}

// The attention output gate: the gate rows are drawn as a linear of their own
// (stream `tid`), so every other weight of a gated model equals the ungated
// model of the same seed, and interleaved per head into q_proj: head h's q
// rows, then its gate rows.  In the .intfer form both halves share the q
// linear's K-group scales (one scale per group for the whole tensor).
bool add_gate_rows(OwnedLinear& q, ifr_linear& L, int nh, int hd, int bits, int group, uint64_t seed,
                   uint64_t tid, bool intfer_form) {
  const int K = L.K, ng = K / group;
  if ((size_t)K * bits % 8 || L.N != nh * hd) return false;
  OwnedLinear g;
  ifr_linear gl;
  make_linear(g, gl, nh * hd, K, bits, group, seed, tid, intfer_form);
  const size_t rb = (size_t)K * bits / 8;
  OwnedLinear o;
  o.codes.resize(2 * q.codes.size());
  o.scale.resize(2 * q.scale.size());
  o.zero.resize(2 * q.zero.size());
  for (int h = 0; h < nh; ++h)
    for (int half = 0; half < 2; ++half) {
      const OwnedLinear& src = half ? g : q;
      const size_t r0 = (size_t)h * hd, d0 = (size_t)(2 * h + half) * hd;
      std::memcpy(&o.codes[d0 * rb], &src.codes[r0 * rb], hd * rb);
      for (size_t r = 0; r < (size_t)hd; ++r)
        for (int gi = 0; gi < ng; ++gi) {
          o.scale[(d0 + r) * ng + gi] = intfer_form ? q.scale[(r0 + r) * ng + gi] : src.scale[(r0 + r) * ng + gi];
          o.zero[(d0 + r) * ng + gi] = src.zero[(r0 + r) * ng + gi];
        }
    }
  q = std::move(o);
  L.N = 2 * nh * hd;
  return true;
}

void round_fp16(std::vector<float>& v) {
  for (float& x : v) x = ifr::h2f(ifr::f2h(x));
}

}  // namespace

extern "C" void ifr_default_cfg(ifr_model_cfg* c) {
  std::memset(c, 0, sizeof(*c));
  c->hidden = 1024;
  c->layers = 28;
  c->n_heads = 16;
  c->n_kv = 8;
  c->head_dim = 128;
  c->inter = 3072;
  c->vocab = 151936;
  c->rotary_dim = 128;
  c->rms_eps = 1e-6f;
  c->rope_theta = 1e6f;
  c->group_size = 128;
  c->qk_norm = 1;
  c->rotate = 1;
}

extern "C" ifr_host_model* ifr_synth_model(const ifr_model_cfg* cfg, uint64_t seed,
                                           int32_t bits_mode) {
  if (!cfg || cfg->hidden <= 0 || cfg->layers <= 0 || cfg->group_size <= 0) return nullptr;
  const bool intfer_form = (bits_mode & IFR_SYNTH_INTFER) != 0;
  bits_mode &= ~IFR_SYNTH_INTFER;
  if (bits_mode != 0 && bits_mode != 2 && bits_mode != 4 && bits_mode != 8) return nullptr;
  auto* m = new OwnedModel();
  m->pub.cfg = *cfg;
  const int H = cfg->hidden, L = cfg->layers, hd = cfg->head_dim;
  const int qN = cfg->n_heads * hd, kvN = cfg->n_kv * hd, F = cfg->inter, G = cfg->group_size;
  m->embed.resize((size_t)cfg->vocab * H);
  fill_normal(m->embed.data(), m->embed.size(), 0.02f, seed, 1);
  m->final_norm.resize(H);
  fill_normal(m->final_norm.data(), H, 0.1f, seed, 2);
  m->layers.resize(L);
  m->norms.resize((size_t)L * 4);
  m->lin.resize((size_t)L * 7);
  uint64_t split = seed ^ 0x5EEDB175ull;
  for (int l = 0; l < L; ++l) {
    ifr_layer_w& w = m->layers[l];
    const int dims[4] = {H, H, hd, hd};
    for (int j = 0; j < 4; ++j) {
      auto& v = m->norms[(size_t)l * 4 + j];
      v.resize(dims[j]);
      fill_normal(v.data(), dims[j], 0.1f, seed, 100 + (uint64_t)l * 8 + j);
      if (intfer_form) round_fp16(v);
    }
    ifr_linear* slots[7] = {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down};
    const int Ns[7] = {qN, kvN, kvN, H, F, F, H};
    const int Ks[7] = {H, H, H, qN, H, H, F};
    for (int j = 0; j < 7; ++j) {
      int bits = bits_mode;
      if (bits_mode == 0) bits = ((splitmix64(split) >> 11) % 10 < 7) ? 2 : 4;
      make_linear(m->lin[(size_t)l * 7 + j], *slots[j], Ns[j], Ks[j], bits, G, seed,
                  1000 + (uint64_t)l * 16 + j, intfer_form);
      if (j == 0 && cfg->attn_gate)
        if (!add_gate_rows(m->lin[(size_t)l * 7], *slots[0], cfg->n_heads, hd, bits, G, seed,
                           1000 + (uint64_t)l * 16 + 7, intfer_form)) {
          delete m;
          return nullptr;
        }
    }
  }
  if (intfer_form) {
    round_fp16(m->embed);
    round_fp16(m->final_norm);
  }
  m->publish();
  return ifrh::adopt(m);
}

extern "C" void ifr_host_model_free(ifr_host_model* p) {
  if (!p) return;
  OwnedModel* m = nullptr;
  {
    std::lock_guard<std::mutex> lk(ifrh::g_models_mu);
    auto it = ifrh::g_models.find(p);
    if (it == ifrh::g_models.end()) return;
    m = it->second;
    ifrh::g_models.erase(it);
  }
  delete m;
}

extern "C" void ifr_synth_free(ifr_host_model* p) { ifr_host_model_free(p); }
