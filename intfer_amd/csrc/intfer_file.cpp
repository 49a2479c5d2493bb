// .intfer model files: the INTFER1 container (a ModelIR and its RotationSet),
// read, written and mapped onto the engine's host model.
//
// Container (reference writer src/quant/output.cpp:396-482, reader :484-595):
//   54-byte little-endian header
//     "INTFER1\0" | u32 version | u32 n_tensors | u64 code_len | u64 scale_len |
//     u64 global_len | u32 n_rotations | u16 reserved | u64 json_len
//   json_len bytes of JSON: {"model_id","n_layers","version","tensors":[...],
//     "rotations":[...]}; a tensor entry carries name, role, N, K, qcfg
//     {scheme, group_size, scale_dtype, has_global_divisor, act, rotation_id},
//     code/scale/global offset+bytes (relative to their regions), est_error;
//     a rotation entry carries id, site, dim, offset (relative to the
//     rotation region, which follows the global region).
//   code region | scale region | global region | fp32 rotation matrices
// Quantized tensors (dashq.cpp:387-402, :531-575, :636-672): codes group-major,
// code index g*N*G + n*Glocal + (k - g*G), packed least-significant bits first;
// one fp16 scale per K-group for all N rows; optional fp32 alpha in the global
// region; value = (fp16(s_g) * alpha) * cb[code] over the canonical codebook
// cb[c] = (2c - C) / C, C = 2^bits - 1.  FP16 tensors hold raw fp16 [N][K].
//
// The JSON writer emits the reference writer's exact bytes for the same
// ModelIR (same key order, no whitespace, integers in decimal, est_error as
// %.9g), so either implementation reads what the other writes.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "host_model.h"
#include "ifr_half.h"
#include "intfer_amd.h"
#include "json_read.h"

using ifrh::fail;
using ifrh::JNode;
using ifrh::JReader;

namespace {

constexpr size_t kHeaderBytes = 8 + 4 + 4 + 8 + 8 + 8 + 4 + 2 + 8;  // 54

// ---- little-endian fields ----------------------------------------------------------
uint32_t ld_u32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
uint64_t ld_u64(const uint8_t* p) { return (uint64_t)ld_u32(p) | (uint64_t)ld_u32(p + 4) << 32; }
uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }
float ld_f32(const uint8_t* p) {
  const uint32_t u = ld_u32(p);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
void st_le(uint8_t* p, uint64_t v, int bytes) {
  for (int i = 0; i < bytes; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

// ---- name tables (quant_spec.h:13-33, spinquant.hpp:45, output.cpp:300-389) ------
const char* const kRoleNames[] = {"EMBED",         "LM_HEAD",         "ATTN_Q",        "ATTN_K",
                                  "ATTN_V",        "ATTN_O",          "MLP_GATE",      "MLP_UP",
                                  "MLP_DOWN",      "NORM",            "ROPE",          "LINEAR_ATTN_QKV",
                                  "LINEAR_ATTN_Z", "LINEAR_ATTN_B",   "LINEAR_ATTN_A", "LINEAR_ATTN_CONV",
                                  "LINEAR_ATTN_OUT", "OTHER"};
constexpr int kRoleOther = 17;
const char* const kSchemeNames[] = {"FP16", "INT8", "INT4", "INT2"};
const char* const kSiteNames[] = {"QKV", "O", "FFN_IN", "FFN_OUT", "NONE"};

int lookup(const char* const* names, int n, const std::string& s, int dflt) {
  for (int i = 0; i < n; ++i)
    if (s == names[i]) return i;
  return dflt;
}
int scheme_bits(int scheme) { return scheme == IFR_SCHEME_INT2 ? 2 : scheme == IFR_SCHEME_INT4 ? 4 : 8; }

// JSON writer fragments: the reference writer's byte format.
void jstr(std::string& o, const std::string& s) {
  o += '"';
  for (const char c : s) {
    const unsigned char u = (unsigned char)c;
    if (c == '"' || c == '\\') { o += '\\'; o += c; }
    else if (c == '\n') o += "\\n";
    else if (c == '\t') o += "\\t";
    else if (c == '\r') o += "\\r";
    else if (u < 0x20) {
      char b[8];
      std::snprintf(b, sizeof(b), "\\u%04x", u);
      o += b;
    } else {
      o += c;
    }
  }
  o += '"';
}
void jkey(std::string& o, const char* k, bool first = false) {
  if (!first) o += ',';
  o += '"';
  o += k;
  o += "\":";
}
void jint(std::string& o, int64_t v) { o += std::to_string(v); }
void jreal(std::string& o, double v) {
  char b[32];
  std::snprintf(b, sizeof(b), "%.9g", v);
  o += b;
}

// ---- canonical Hadamard --------------------------------------------------------------
uint32_t floor_pow2(uint32_t n) {
  uint32_t p = 1;
  while (p * 2 <= n && p * 2 != 0) p *= 2;
  return p;
}
// Entry (i, j) of the canonical rotation of `dim`: Sylvester H_p / sqrt(p) on
// the leading p x p block (H(i,j) = (-1)^popcount(i & j)), identity after it
// (spinquant.cpp:82-125).
float hadamard_entry(uint32_t dim, uint32_t i, uint32_t j) {
  const uint32_t p = floor_pow2(dim);
  if (i < p && j < p) {
    const float s = 1.0f / std::sqrt((float)p);
    return (__builtin_popcount(i & j) & 1) ? -s : s;
  }
  return (i == j) ? 1.0f : 0.0f;
}
// The reference's shape check (spinquant.cpp:607-629) tolerates 1e-6 on the
// magnitudes but ignores signs; this one also demands the Sylvester signs,
// since the online replay applies exactly the FWHT.
bool is_canonical_hadamard(const uint8_t* mat, uint32_t dim) {
  if (dim == 0) return false;
  for (uint32_t i = 0; i < dim; ++i)
    for (uint32_t j = 0; j < dim; ++j) {
      const float v = ld_f32(mat + ((size_t)i * dim + j) * 4);
      if (!(std::fabs(v - hadamard_entry(dim, i, j)) <= 1e-6f)) return false;
    }
  return true;
}

struct ITensor {
  std::string name;
  int role = kRoleOther;
  uint32_t N = 0, K = 0;
  int scheme = IFR_SCHEME_FP16;
  uint16_t group = 0;
  int scale_dtype = 0;
  bool has_global = false;
  int act = 0;
  uint8_t rot_id = 0;
  uint64_t code_off = 0, code_bytes = 0, scale_off = 0, scale_bytes = 0, global_off = 0, global_bytes = 0;
  float est_error = 0.f;
};

struct IRotation {
  uint8_t id = 0;
  int site = IFR_SITE_NONE;
  uint32_t dim = 0;
  const uint8_t* mat = nullptr;  // dim*dim little-endian fp32
  bool hadamard = false;
};

bool slice_ok(uint64_t off, uint64_t bytes, uint64_t len) { return off <= len && bytes <= len - off; }

}  // namespace

struct ifr_intfer {
  const uint8_t* base = nullptr;
  size_t n = 0;
  std::string model_id;
  uint32_t n_layers = 0;
  std::vector<ITensor> tensors;
  std::vector<IRotation> rotations;
  const uint8_t *code = nullptr, *scale = nullptr, *global = nullptr;
  uint64_t code_len = 0, scale_len = 0, global_len = 0;
};

namespace {

int parse(const uint8_t* d, size_t n, ifr_intfer& f) {
  if (n < kHeaderBytes) return fail(IFR_EINVAL, "intfer: %zu bytes, shorter than the header", n);
  if (std::memcmp(d, "INTFER1", 7) != 0) return fail(IFR_EINVAL, "intfer: bad magic");
  const uint32_t n_tensors = ld_u32(d + 12);
  const uint64_t code_len = ld_u64(d + 16), scale_len = ld_u64(d + 24), global_len = ld_u64(d + 32);
  const uint32_t n_rot = ld_u32(d + 40);
  const uint64_t json_len = ld_u64(d + 46);
  size_t pos = kHeaderBytes;
  if (json_len > n - pos) return fail(IFR_EINVAL, "intfer: JSON runs past the end");
  JNode root;
  JReader rd(reinterpret_cast<const char*>(d + pos), reinterpret_cast<const char*>(d + pos + json_len));
  if (!rd.document(root) || root.kind != JNode::Obj) return fail(IFR_EINVAL, "intfer: malformed JSON");
  pos += json_len;
  if (const JNode* v = root.at("model_id", JNode::Str)) f.model_id = v->s;
  if (const JNode* v = root.at("n_layers", JNode::Int)) f.n_layers = (uint32_t)v->i;

  const JNode* jt = root.at("tensors", JNode::Arr);
  if (!jt) return fail(IFR_EINVAL, "intfer: no tensors array");
  if (jt->items.size() != n_tensors)
    return fail(IFR_EINVAL, "intfer: header says %u tensors, JSON has %zu", n_tensors, jt->items.size());
  f.tensors.reserve(n_tensors);
  for (const JNode& o : jt->items) {
    if (o.kind != JNode::Obj) return fail(IFR_EINVAL, "intfer: tensor entry is not an object");
    ITensor t;
    if (const JNode* v = o.at("name", JNode::Str)) t.name = v->s;
    if (const JNode* v = o.at("role", JNode::Str)) t.role = lookup(kRoleNames, 18, v->s, kRoleOther);
    if (const JNode* v = o.at("N", JNode::Int)) t.N = (uint32_t)v->i;
    if (const JNode* v = o.at("K", JNode::Int)) t.K = (uint32_t)v->i;
    if (const JNode* q = o.at("qcfg", JNode::Obj)) {
      if (const JNode* v = q->at("scheme", JNode::Str)) t.scheme = lookup(kSchemeNames, 4, v->s, IFR_SCHEME_FP16);
      if (const JNode* v = q->at("group_size", JNode::Int)) t.group = (uint16_t)v->i;
      if (const JNode* v = q->at("scale_dtype", JNode::Str)) t.scale_dtype = v->s == "FP8_E4M3" ? 1 : 0;
      if (const JNode* v = q->at("has_global_divisor", JNode::Bool)) t.has_global = v->b;
      if (const JNode* v = q->at("act", JNode::Str)) t.act = v->s == "BF16" ? 1 : v->s == "INT8_G64" ? 2 : 0;
      if (const JNode* v = q->at("rotation_id", JNode::Int)) t.rot_id = (uint8_t)v->i;
    }
    auto u64 = [&](const char* k) -> uint64_t {
      const JNode* v = o.at(k, JNode::Int);
      return v ? (uint64_t)v->i : 0;
    };
    t.code_off = u64("code_offset");
    t.code_bytes = u64("code_bytes");
    t.scale_off = u64("scale_offset");
    t.scale_bytes = u64("scale_bytes");
    t.global_off = u64("global_offset");
    t.global_bytes = u64("global_bytes");
    if (const JNode* v = o.at("est_error", JNode::Real)) t.est_error = (float)v->d;
    if (!slice_ok(t.code_off, t.code_bytes, code_len) || !slice_ok(t.scale_off, t.scale_bytes, scale_len) ||
        !slice_ok(t.global_off, t.global_bytes, global_len))
      return fail(IFR_EINVAL, "intfer: tensor '%s' has a slice outside its region", t.name.c_str());
    f.tensors.push_back(std::move(t));
  }
  if (code_len > n - pos || scale_len > n - pos - code_len || global_len > n - pos - code_len - scale_len)
    return fail(IFR_EINVAL, "intfer: payload regions run past the end");
  f.code = d + pos;
  f.scale = f.code + code_len;
  f.global = f.scale + scale_len;
  f.code_len = code_len;
  f.scale_len = scale_len;
  f.global_len = global_len;
  pos += code_len + scale_len + global_len;

  const JNode* jr = root.at("rotations", JNode::Arr);
  if (!jr) return fail(IFR_EINVAL, "intfer: no rotations array");
  if (jr->items.size() != n_rot)
    return fail(IFR_EINVAL, "intfer: header says %u rotations, JSON has %zu", n_rot, jr->items.size());
  for (const JNode& o : jr->items) {
    if (o.kind != JNode::Obj) return fail(IFR_EINVAL, "intfer: rotation entry is not an object");
    IRotation r;
    uint64_t off = 0;
    if (const JNode* v = o.at("id", JNode::Int)) r.id = (uint8_t)v->i;
    if (const JNode* v = o.at("site", JNode::Str)) r.site = lookup(kSiteNames, 4, v->s, IFR_SITE_NONE);
    if (const JNode* v = o.at("dim", JNode::Int)) r.dim = (uint32_t)v->i;
    if (const JNode* v = o.at("offset", JNode::Int)) off = (uint64_t)v->i;
    const uint64_t bytes = (uint64_t)r.dim * r.dim * 4;
    if (r.dim > 65536 || !slice_ok(off, bytes, n - pos))
      return fail(IFR_EINVAL, "intfer: rotation %u matrix runs past the end", (unsigned)r.id);
    r.mat = d + pos + off;
    r.hadamard = is_canonical_hadamard(r.mat, r.dim);
    f.rotations.push_back(r);
  }
  f.base = d;
  f.n = n;
  return IFR_OK;
}

// Dequantize one tensor (QuantResult::dequant, dashq.cpp:531-575).
int dequant(const ifr_intfer& f, const ITensor& t, float* out) {
  const size_t NK = (size_t)t.N * t.K;
  const uint8_t* code = f.code + t.code_off;
  if (t.scheme == IFR_SCHEME_FP16) {
    if (t.code_bytes < NK * 2) return fail(IFR_EINVAL, "intfer: '%s' FP16 payload too short", t.name.c_str());
    for (size_t i = 0; i < NK; ++i) out[i] = ifr::h2f(ld_u16(code + 2 * i));
    return IFR_OK;
  }
  if (t.scale_dtype != 0)
    return fail(IFR_EDECLINE, "intfer: '%s' has FP8 scales (the quantizer writes FP16)", t.name.c_str());
  const int bits = scheme_bits(t.scheme);
  const int C = (1 << bits) - 1;
  const uint32_t G = t.group > 0 ? t.group : t.K;
  const uint32_t ngr = G ? (t.K + G - 1) / G : 0;
  if (t.scale_bytes < (uint64_t)ngr * 2)
    return fail(IFR_EINVAL, "intfer: '%s' has %llu scale bytes for %u groups", t.name.c_str(),
                (unsigned long long)t.scale_bytes, ngr);
  if (t.global_bytes > 0 && t.global_bytes < 4)
    return fail(IFR_EINVAL, "intfer: '%s' global divisor of %llu bytes", t.name.c_str(),
                (unsigned long long)t.global_bytes);
  if (ngr > 0) {
    const uint32_t gl = ngr - 1, last = t.K - gl * G;
    const uint64_t ncodes = (uint64_t)gl * t.N * G + (uint64_t)t.N * last;
    if (t.code_bytes * 8 < ncodes * bits)
      return fail(IFR_EINVAL, "intfer: '%s' code payload too short", t.name.c_str());
  }
  const float alpha = t.global_bytes >= 4 ? ld_f32(f.global + t.global_off) : 1.0f;
  float cb[256];
  for (int c = 0; c <= C; ++c) cb[c] = (2.0f * (float)c - (float)C) / (float)C;
  const uint8_t* sc = f.scale + t.scale_off;
  for (uint32_t g = 0; g < ngr; ++g) {
    const float s = ifr::h2f(ld_u16(sc + 2 * g)) * alpha;
    const uint32_t k0 = g * G, gl = std::min(t.K, k0 + G) - k0;
    for (uint32_t r = 0; r < t.N; ++r) {
      const uint64_t base = (uint64_t)g * t.N * G + (uint64_t)r * gl;
      for (uint32_t c = 0; c < gl; ++c) {
        const uint64_t i = base + c;
        const int v = bits == 8 ? code[i] : (code[i * bits / 8] >> ((i * bits) % 8)) & C;
        out[(size_t)r * t.K + k0 + c] = s * cb[v];
      }
    }
  }
  return IFR_OK;
}

// ---- mapping to the host model -------------------------------------------------------
struct Mapper {
  const ifr_intfer& f;
  ifr_model_cfg cfg;
  std::map<std::string, size_t> by_name;  // last entry of a repeated name
  std::map<uint8_t, const IRotation*> by_id;
  int rotated = 0, plain = 0;

  explicit Mapper(const ifr_intfer& file, const ifr_model_cfg& c) : f(file), cfg(c) {
    for (size_t i = 0; i < f.tensors.size(); ++i) by_name[f.tensors[i].name] = i;
    for (const IRotation& r : f.rotations) by_id[r.id] = &r;  // a later id replaces an earlier one
  }
  const ITensor* find(const std::string& n) const {
    auto it = by_name.find(n);
    return it == by_name.end() ? nullptr : &f.tensors[it->second];
  }
  int need(const std::string& n, const ITensor** t) const {
    *t = find(n);
    return *t ? IFR_OK : fail(IFR_EINVAL, "intfer: missing tensor %s", n.c_str());
  }
  // A host fp32 tensor of `elems` values (any scheme, dequantized).
  int host(const ITensor& t, size_t elems, std::vector<float>& out) const {
    if ((size_t)t.N * t.K != elems)
      return fail(IFR_EINVAL, "intfer: %s is %ux%u, expected %zu values", t.name.c_str(), t.N, t.K, elems);
    out.resize(elems);
    return dequant(f, t, out.data());
  }
  int linear(const ITensor& t, int N, int K, bool left_site, ifr_linear& L, ifrh::OwnedLinear& o) {
    if (t.scheme == IFR_SCHEME_FP16)
      return fail(IFR_EDECLINE, "intfer: %s is FP16; linears run on the int8 GEMM only", t.name.c_str());
    if (t.scale_dtype != 0) return fail(IFR_EDECLINE, "intfer: %s has FP8 scales", t.name.c_str());
    const uint32_t G = t.group > 0 ? t.group : t.K;
    if (G != 128) return fail(IFR_EDECLINE, "intfer: %s group %u, the GEMM needs 128", t.name.c_str(), G);
    if ((int)t.N != N || (int)t.K != K)
      return fail(IFR_EINVAL, "intfer: %s is %ux%u, the config needs %dx%d", t.name.c_str(), t.N, t.K, N, K);
    const int bits = scheme_bits(t.scheme), C = (1 << bits) - 1, ng = K / 128;
    const size_t row_bytes = (size_t)K * bits / 8, seg = (size_t)128 * bits / 8;
    if (t.code_bytes < (size_t)N * row_bytes) return fail(IFR_EINVAL, "intfer: %s code payload too short", t.name.c_str());
    if (t.scale_bytes < (uint64_t)ng * 2) return fail(IFR_EINVAL, "intfer: %s scale payload too short", t.name.c_str());
    if (t.global_bytes > 0 && t.global_bytes < 4)
      return fail(IFR_EINVAL, "intfer: %s global divisor of %llu bytes", t.name.c_str(),
                  (unsigned long long)t.global_bytes);
    const float alpha = t.global_bytes >= 4 ? ld_f32(f.global + t.global_off) : 1.0f;
    if (!std::isfinite(alpha)) return fail(IFR_EINVAL, "intfer: %s alpha not finite", t.name.c_str());
    // Group-major (g, n) runs of 128 codes are whole bytes at every width, so
    // each run moves to its row-major place (n, g) with one copy.
    const uint8_t* src = f.code + t.code_off;
    o.codes.assign((size_t)N * row_bytes, 0);
    for (int g = 0; g < ng; ++g)
      for (int n = 0; n < N; ++n)
        std::memcpy(&o.codes[(size_t)n * row_bytes + g * seg], src + ((size_t)g * N + n) * seg, seg);
    const uint8_t* sc = f.scale + t.scale_off;
    o.scale.resize((size_t)N * ng);
    o.zero.assign((size_t)N * ng, ifr::f2h((float)C * 0.5f));
    for (int n = 0; n < N; ++n)
      for (int g = 0; g < ng; ++g) o.scale[(size_t)n * ng + g] = ld_u16(sc + 2 * g);
    L.N = N;
    L.K = K;
    L.bits = bits;
    L.group = 128;
    L.post = (2.0f * alpha) / (float)C;
    // Rotation replay: by rotation_id (main.cpp:839-850); the engine's FWHT
    // replays exactly the canonical Hadamard of the hidden size.
    auto it = by_id.find(t.rot_id);
    if (it == by_id.end()) {
      ++plain;
      return IFR_OK;
    }
    const IRotation& R = *it->second;
    const uint32_t dim = left_site ? t.N : t.K;
    if (!R.hadamard) return fail(IFR_EDECLINE, "intfer: %s uses dense rotation %u", t.name.c_str(), R.id);
    if (R.dim != dim || (int)dim != cfg.hidden)
      return fail(IFR_EDECLINE, "intfer: %s rotation dim %u, expected %u", t.name.c_str(), R.dim, dim);
    ++rotated;
    return IFR_OK;
  }
};

int build_host(const ifr_intfer& f, const ifr_model_cfg& cfg_in, ifr_host_model** out) {
  ifr_model_cfg cfg = cfg_in;
  const int H = cfg.hidden, Lc = cfg.layers, hd = cfg.head_dim, V = cfg.vocab;
  if (H <= 0 || Lc <= 0 || hd <= 0 || cfg.n_heads <= 0 || cfg.n_kv <= 0 || cfg.inter <= 0 || V <= 0)
    return fail(IFR_EINVAL, "intfer: config dimensions must be positive");
  if (f.n_layers != 0 && (int)f.n_layers != Lc)
    return fail(IFR_EINVAL, "intfer: file has %u layers, the config %d", f.n_layers, Lc);
  const int qN = cfg.n_heads * hd, kvN = cfg.n_kv * hd, F = cfg.inter;
  Mapper mp(f, cfg);
  std::unique_ptr<ifrh::OwnedModel> m(new ifrh::OwnedModel());
  const std::string pre = "model.language_model.";
  const ITensor* t = nullptr;
  if (int r = mp.need(pre + "embed_tokens.weight", &t)) return r;
  if (int r = mp.host(*t, (size_t)V * H, m->embed)) return r;
  if (int r = mp.need(pre + "norm.weight", &t)) return r;
  if (int r = mp.host(*t, H, m->final_norm)) return r;
  t = mp.find("lm_head.weight");
  if (!t) t = mp.find(pre + "lm_head.weight");
  if (t)
    if (int r = mp.host(*t, (size_t)V * H, m->lm_head)) return r;
  m->norms.resize((size_t)Lc * 4);
  m->lin.resize((size_t)Lc * 7);
  m->layers.resize(Lc);
  static const char* const kNorms[4] = {"input_layernorm", "post_attention_layernorm", "self_attn.q_norm",
                                        "self_attn.k_norm"};
  static const char* const kLin[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                      "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                                      "mlp.down_proj"};
  int Ns[7] = {qN, kvN, kvN, H, F, F, H};
  const int Ks[7] = {H, H, H, qN, H, H, F};
  const bool left[7] = {false, false, false, true, false, false, true};
  // the attention output gate is set from the file, as the reference decides
  // packed_gate from the q projection's size (main.cpp:7624): q_proj with
  // 2 * n_heads * head_dim rows carries [q, gate] per head
  cfg.attn_gate = 0;
  {
    if (int r = mp.need(pre + "layers.0.self_attn.q_proj.weight", &t)) return r;
    if ((int)t->N == 2 * qN) cfg.attn_gate = 1;
    Ns[0] = cfg.attn_gate ? 2 * qN : qN;
  }
  for (int l = 0; l < Lc; ++l) {
    const std::string lp = pre + "layers." + std::to_string(l) + ".";
    for (int j = 0; j < 4; ++j) {
      if (j >= 2 && !cfg.qk_norm) continue;
      if (int r = mp.need(lp + kNorms[j] + ".weight", &t)) return r;
      if (int r = mp.host(*t, j < 2 ? H : hd, m->norms[(size_t)l * 4 + j])) return r;
    }
    ifr_layer_w& w = m->layers[l];
    ifr_linear* slots[7] = {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down};
    for (int j = 0; j < 7; ++j) {
      if (int r = mp.need(lp + kLin[j] + ".weight", &t)) return r;
      if (int r = mp.linear(*t, Ns[j], Ks[j], left[j], *slots[j], m->lin[(size_t)l * 7 + j])) return r;
    }
  }
  if (mp.rotated && mp.plain)
    return fail(IFR_EDECLINE, "intfer: %d linears rotated, %d not; the engine rotates all or none",
                mp.rotated, mp.plain);
  cfg.rotate = mp.rotated > 0 ? 1 : 0;
  cfg.group_size = 128;
  m->pub.cfg = cfg;
  m->publish();
  *out = ifrh::adopt(m.release());
  return IFR_OK;
}

// ---- writer ----------------------------------------------------------------------------
struct WTensor {
  std::string name;
  int role = kRoleOther;
  uint32_t N = 0, K = 0;
  int scheme = IFR_SCHEME_FP16;
  int group = 0;
  bool has_global = false;
  float alpha = 1.0f;
  int rot_id = 0;
  const float* f32 = nullptr;      // FP16 tensors: source values
  const ifr_linear* lin = nullptr;  // quantized tensors
  uint64_t code_off = 0, code_bytes = 0, scale_off = 0, scale_bytes = 0, global_off = 0, global_bytes = 0;
};

float post_of(const ifr_linear& w) { return w.post == 0.0f ? 1.0f : w.post; }

// Whether a host linear has the container's form; sets alpha.
int check_container_form(const ifr_linear& w, const std::string& name, float* alpha) {
  if (!w.codes || !w.scale || !w.zero) return fail(IFR_EINVAL, "intfer write: %s has a null buffer", name.c_str());
  if (w.bits != 2 && w.bits != 4 && w.bits != 8) return fail(IFR_EDECLINE, "intfer write: %s bits %d", name.c_str(), w.bits);
  if (w.group != 128 || w.N <= 0 || w.K <= 0 || w.K % 128)
    return fail(IFR_EDECLINE, "intfer write: %s needs group 128 and K %% 128 == 0", name.c_str());
  const int C = (1 << w.bits) - 1, ng = w.K / 128;
  const uint16_t z = ifr::f2h((float)C * 0.5f);
  for (int n = 0; n < w.N; ++n)
    for (int g = 0; g < ng; ++g) {
      const size_t i = (size_t)n * ng + g;
      if (w.zero[i] != z || w.scale[i] != w.scale[g])
        return fail(IFR_EDECLINE, "intfer write: %s has per-row scales or a zero other than C/2", name.c_str());
    }
  const float post = post_of(w);
  const float a = post * ((float)C * 0.5f);
  if (!std::isfinite(a) || (2.0f * a) / (float)C != post)
    return fail(IFR_EDECLINE, "intfer write: %s post %g is not 2*alpha/C for an fp32 alpha", name.c_str(), post);
  *alpha = a;
  return IFR_OK;
}

int write_model(const ifr_host_model& m, const char* model_id, void** out, size_t* out_n) {
  const ifr_model_cfg& c = m.cfg;
  const int H = c.hidden, L = c.layers, hd = c.head_dim, V = c.vocab;
  if (!m.embed || !m.final_norm || !m.layers || H <= 0 || L <= 0 || V <= 0 || hd <= 0)
    return fail(IFR_EINVAL, "intfer write: incomplete host model");
  std::vector<WTensor> ts;
  const std::string pre = "model.language_model.";
  auto add_f16 = [&](const std::string& name, int role, uint32_t N, uint32_t K, const float* v) {
    WTensor t;
    t.name = name;
    t.role = role;
    t.N = N;
    t.K = K;
    t.f32 = v;
    ts.push_back(std::move(t));
  };
  auto add_lin = [&](const std::string& name, int role, const ifr_linear& w, int site) -> int {
    WTensor t;
    t.name = name;
    t.role = role;
    t.N = (uint32_t)w.N;
    t.K = (uint32_t)w.K;
    if (int r = check_container_form(w, name, &t.alpha)) return r;
    t.scheme = w.bits == 2 ? IFR_SCHEME_INT2 : w.bits == 4 ? IFR_SCHEME_INT4 : IFR_SCHEME_INT8;
    t.group = 128;
    t.has_global = t.alpha != 1.0f;
    t.rot_id = c.rotate ? 1 + site : 0;
    t.lin = &w;
    ts.push_back(std::move(t));
    return IFR_OK;
  };
  add_f16(pre + "embed_tokens.weight", IFR_ROLE_EMBED, V, H, m.embed);
  for (int l = 0; l < L; ++l) {
    const ifr_layer_w& w = m.layers[l];
    const std::string lp = pre + "layers." + std::to_string(l) + ".";
    if (!w.in_ln || !w.post_ln) return fail(IFR_EINVAL, "intfer write: layer %d norms missing", l);
    add_f16(lp + "input_layernorm.weight", IFR_ROLE_NORM, H, 1, w.in_ln);
    int r = add_lin(lp + "self_attn.q_proj.weight", IFR_ROLE_ATTN_Q, w.q, IFR_SITE_QKV);
    if (!r) r = add_lin(lp + "self_attn.k_proj.weight", IFR_ROLE_ATTN_K, w.k, IFR_SITE_QKV);
    if (!r) r = add_lin(lp + "self_attn.v_proj.weight", IFR_ROLE_ATTN_V, w.v, IFR_SITE_QKV);
    if (!r) r = add_lin(lp + "self_attn.o_proj.weight", IFR_ROLE_ATTN_O, w.o, IFR_SITE_O);
    if (r) return r;
    if (c.qk_norm) {
      if (!w.q_norm || !w.k_norm) return fail(IFR_EINVAL, "intfer write: layer %d q/k norms missing", l);
      add_f16(lp + "self_attn.q_norm.weight", IFR_ROLE_NORM, hd, 1, w.q_norm);
      add_f16(lp + "self_attn.k_norm.weight", IFR_ROLE_NORM, hd, 1, w.k_norm);
    }
    add_f16(lp + "post_attention_layernorm.weight", IFR_ROLE_NORM, H, 1, w.post_ln);
    r = add_lin(lp + "mlp.gate_proj.weight", IFR_ROLE_MLP_GATE, w.gate, IFR_SITE_FFN_IN);
    if (!r) r = add_lin(lp + "mlp.up_proj.weight", IFR_ROLE_MLP_UP, w.up, IFR_SITE_FFN_IN);
    if (!r) r = add_lin(lp + "mlp.down_proj.weight", IFR_ROLE_MLP_DOWN, w.down, IFR_SITE_FFN_OUT);
    if (r) return r;
  }
  add_f16(pre + "norm.weight", IFR_ROLE_NORM, H, 1, m.final_norm);
  if (m.lm_head) add_f16("lm_head.weight", IFR_ROLE_LM_HEAD, V, H, m.lm_head);

  uint64_t code_len = 0, scale_len = 0, global_len = 0;
  for (WTensor& t : ts) {
    t.code_off = code_len;
    t.scale_off = scale_len;
    t.global_off = global_len;
    if (t.scheme == IFR_SCHEME_FP16) {
      t.code_bytes = (uint64_t)t.N * t.K * 2;
    } else {
      t.code_bytes = (uint64_t)t.N * t.K * scheme_bits(t.scheme) / 8;
      t.scale_bytes = (uint64_t)(t.K / 128) * 2;
      t.global_bytes = t.has_global ? 4 : 0;
    }
    code_len += t.code_bytes;
    scale_len += t.scale_bytes;
    global_len += t.global_bytes;
  }
  const int n_rot = c.rotate ? 4 : 0;

  std::string js;
  jkey(js += '{', "model_id", true);
  jstr(js, model_id ? model_id : "");
  jkey(js, "n_layers");
  jint(js, L);
  jkey(js, "version");
  jint(js, 1);
  jkey(js, "tensors");
  js += '[';
  for (size_t i = 0; i < ts.size(); ++i) {
    const WTensor& t = ts[i];
    if (i) js += ',';
    jkey(js += '{', "name", true);
    jstr(js, t.name);
    jkey(js, "role");
    jstr(js, kRoleNames[t.role]);
    jkey(js, "N");
    jint(js, t.N);
    jkey(js, "K");
    jint(js, t.K);
    jkey(js, "qcfg");
    jkey(js += '{', "scheme", true);
    jstr(js, kSchemeNames[t.scheme]);
    jkey(js, "group_size");
    jint(js, t.group);
    jkey(js, "scale_dtype");
    jstr(js, "FP16");
    jkey(js, "has_global_divisor");
    js += t.has_global ? "true" : "false";
    jkey(js, "act");
    jstr(js, "FP16");
    jkey(js, "rotation_id");
    jint(js, t.rot_id);
    js += '}';
    jkey(js, "code_offset");
    jint(js, (int64_t)t.code_off);
    jkey(js, "code_bytes");
    jint(js, (int64_t)t.code_bytes);
    jkey(js, "scale_offset");
    jint(js, (int64_t)t.scale_off);
    jkey(js, "scale_bytes");
    jint(js, (int64_t)t.scale_bytes);
    jkey(js, "global_offset");
    jint(js, (int64_t)t.global_off);
    jkey(js, "global_bytes");
    jint(js, (int64_t)t.global_bytes);
    jkey(js, "est_error");
    jreal(js, 0.0);
    js += '}';
  }
  js += ']';
  jkey(js, "rotations");
  js += '[';
  for (int k = 0; k < n_rot; ++k) {
    if (k) js += ',';
    jkey(js += '{', "id", true);
    jint(js, 1 + k);
    jkey(js, "site");
    jstr(js, kSiteNames[k]);
    jkey(js, "dim");
    jint(js, H);
    jkey(js, "offset");
    jint(js, (int64_t)k * H * H * 4);
    js += '}';
  }
  js += "]}";

  const uint64_t rot_bytes = (uint64_t)n_rot * H * H * 4;
  const uint64_t total = kHeaderBytes + js.size() + code_len + scale_len + global_len + rot_bytes;
  uint8_t* buf = static_cast<uint8_t*>(std::malloc(total));
  if (!buf) return fail(IFR_ENOMEM, "intfer write: %llu bytes", (unsigned long long)total);
  std::memcpy(buf, "INTFER1", 8);
  st_le(buf + 8, 1, 4);
  st_le(buf + 12, ts.size(), 4);
  st_le(buf + 16, code_len, 8);
  st_le(buf + 24, scale_len, 8);
  st_le(buf + 32, global_len, 8);
  st_le(buf + 40, (uint64_t)n_rot, 4);
  st_le(buf + 44, 0, 2);
  st_le(buf + 46, js.size(), 8);
  std::memcpy(buf + kHeaderBytes, js.data(), js.size());
  uint8_t* code = buf + kHeaderBytes + js.size();
  uint8_t* scale = code + code_len;
  uint8_t* global = scale + scale_len;
  uint8_t* rot = global + global_len;
  for (const WTensor& t : ts) {
    if (t.scheme == IFR_SCHEME_FP16) {
      const size_t nk = (size_t)t.N * t.K;
      uint8_t* p = code + t.code_off;
      for (size_t i = 0; i < nk; ++i) st_le(p + 2 * i, ifr::f2h(t.f32[i]), 2);
      continue;
    }
    const ifr_linear& w = *t.lin;
    const int ng = w.K / 128;
    const size_t row_bytes = (size_t)w.K * w.bits / 8, seg = (size_t)128 * w.bits / 8;
    uint8_t* p = code + t.code_off;
    for (int g = 0; g < ng; ++g)
      for (int n = 0; n < w.N; ++n)
        std::memcpy(p + ((size_t)g * w.N + n) * seg, w.codes + (size_t)n * row_bytes + g * seg, seg);
    for (int g = 0; g < ng; ++g) st_le(scale + t.scale_off + 2 * g, w.scale[g], 2);
    if (t.has_global) {
      uint32_t u;
      std::memcpy(&u, &t.alpha, 4);
      st_le(global + t.global_off, u, 4);
    }
  }
  for (int k = 0; k < n_rot; ++k)
    for (int i = 0; i < H; ++i)
      for (int j = 0; j < H; ++j) {
        const float v = hadamard_entry((uint32_t)H, (uint32_t)i, (uint32_t)j);
        uint32_t u;
        std::memcpy(&u, &v, 4);
        st_le(rot + (((size_t)k * H + i) * H + j) * 4, u, 4);
      }
  *out = buf;
  *out_n = (size_t)total;
  return IFR_OK;
}

}  // namespace

extern "C" {

int ifr_intfer_open(const void* blob, size_t n, ifr_intfer** out) {
  if (!blob || !out) return fail(IFR_EINVAL, "null arg");
  std::unique_ptr<ifr_intfer> f(new ifr_intfer());
  if (int r = parse(static_cast<const uint8_t*>(blob), n, *f)) return r;
  *out = f.release();
  return IFR_OK;
}

int ifr_intfer_close(ifr_intfer* f) {
  delete f;
  return IFR_OK;
}

int ifr_intfer_counts(const ifr_intfer* f, int32_t* n_tensors, int32_t* n_rotations, int32_t* n_layers) {
  if (!f) return fail(IFR_EINVAL, "null arg");
  if (n_tensors) *n_tensors = (int32_t)f->tensors.size();
  if (n_rotations) *n_rotations = (int32_t)f->rotations.size();
  if (n_layers) *n_layers = (int32_t)f->n_layers;
  return IFR_OK;
}

int ifr_intfer_model_id(const ifr_intfer* f, char* buf, size_t cap) {
  if (!f || !buf || cap == 0) return fail(IFR_EINVAL, "null arg");
  const size_t n = std::min(cap - 1, f->model_id.size());
  std::memcpy(buf, f->model_id.data(), n);
  buf[n] = 0;
  return IFR_OK;
}

int ifr_intfer_tensor_info(const ifr_intfer* f, int32_t i, ifr_intfer_tensor* out) {
  if (!f || !out) return fail(IFR_EINVAL, "null arg");
  if (i < 0 || (size_t)i >= f->tensors.size()) return fail(IFR_EINVAL, "tensor index %d", i);
  const ITensor& t = f->tensors[i];
  out->name = t.name.c_str();
  out->role = t.role;
  out->N = (int32_t)t.N;
  out->K = (int32_t)t.K;
  out->scheme = t.scheme;
  out->group_size = t.group;
  out->scale_dtype = t.scale_dtype;
  out->has_global_divisor = t.has_global ? 1 : 0;
  out->act = t.act;
  out->rotation_id = t.rot_id;
  out->code_offset = t.code_off;
  out->code_bytes = t.code_bytes;
  out->scale_offset = t.scale_off;
  out->scale_bytes = t.scale_bytes;
  out->global_offset = t.global_off;
  out->global_bytes = t.global_bytes;
  out->est_error = t.est_error;
  return IFR_OK;
}

int ifr_intfer_find(const ifr_intfer* f, const char* name, int32_t* index) {
  if (!f || !name || !index) return fail(IFR_EINVAL, "null arg");
  for (size_t i = f->tensors.size(); i-- > 0;)
    if (f->tensors[i].name == name) {
      *index = (int32_t)i;
      return IFR_OK;
    }
  return fail(IFR_EINVAL, "no tensor named %s", name);
}

int ifr_intfer_rotation_info(const ifr_intfer* f, int32_t i, ifr_intfer_rotation* out, float* mat) {
  if (!f || !out) return fail(IFR_EINVAL, "null arg");
  if (i < 0 || (size_t)i >= f->rotations.size()) return fail(IFR_EINVAL, "rotation index %d", i);
  const IRotation& r = f->rotations[i];
  out->id = r.id;
  out->site = r.site;
  out->dim = (int32_t)r.dim;
  out->hadamard = r.hadamard ? 1 : 0;
  if (mat)
    for (size_t k = 0; k < (size_t)r.dim * r.dim; ++k) mat[k] = ld_f32(r.mat + 4 * k);
  return IFR_OK;
}

int ifr_intfer_dequant(const ifr_intfer* f, int32_t i, float* out) {
  if (!f || !out) return fail(IFR_EINVAL, "null arg");
  if (i < 0 || (size_t)i >= f->tensors.size()) return fail(IFR_EINVAL, "tensor index %d", i);
  return dequant(*f, f->tensors[i], out);
}

int ifr_intfer_host_model(const ifr_intfer* f, const ifr_model_cfg* cfg, ifr_host_model** out) {
  if (!f || !cfg || !out) return fail(IFR_EINVAL, "null arg");
  return build_host(*f, *cfg, out);
}

int ifr_intfer_write(const ifr_host_model* m, const char* model_id, void** out, size_t* n) {
  if (!m || !out || !n) return fail(IFR_EINVAL, "null arg");
  return write_model(*m, model_id, out, n);
}

void ifr_intfer_buffer_free(void* p) { std::free(p); }

int ifr_model_load_intfer(ifr_ctx* ctx, const void* blob, size_t n, const ifr_model_cfg* cfg,
                          const ifr_kv_cfg* kv) {
  if (!ctx || !blob || !cfg || !kv) return fail(IFR_EINVAL, "null arg");
  ifr_intfer* f = nullptr;
  if (int r = ifr_intfer_open(blob, n, &f)) return r;
  ifr_host_model* m = nullptr;
  int r = ifr_intfer_host_model(f, cfg, &m);
  ifr_intfer_close(f);
  if (r) return r;
  r = ifr_model_load(ctx, m, kv);
  ifr_host_model_free(m);
  return r;
}

int ifr_model_load_intfer_file(ifr_ctx* ctx, const char* path, const ifr_model_cfg* cfg,
                               const ifr_kv_cfg* kv) {
  if (!ctx || !path || !cfg || !kv) return fail(IFR_EINVAL, "null arg");
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(IFR_EINVAL, "cannot open %s", path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    return fail(IFR_EINVAL, "cannot stat %s", path);
  }
  void* p = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) return fail(IFR_ENOMEM, "cannot map %s", path);
  const int r = ifr_model_load_intfer(ctx, p, (size_t)st.st_size, cfg, kv);
  ::munmap(p, (size_t)st.st_size);
  return r;
}

}  // extern "C"
