// CPU ORACLE PIN -- test infrastructure only.
//
// extern "C" entry points over the reference's own host quant core, compiled
// from the sources where they lie under the reference root (see
// oracle/Makefile, target `ref`).  The output library lives in oracle/_ref/
// (git-ignored) and is used only by tests/ to pin the oracle restatement
// against the reference's code: fp16 conversion (src/quant/dashq.cpp:338-384),
// act-quant (dashq.cpp:221-336), the canonical codebook + dequant
// (dashq.cpp:405-417, :531-575), the FWHT rotation (src/spinquant.cpp:99-125,
// :303-312, :586-629) and the INTFER1 container (src/quant/output.cpp:396-603).
#include <cstdint>
#include <cstring>
#include <vector>

#include <cstdlib>

#include "intfer/output.hpp"
#include "intfer/quant/dashq.hpp"
#include "intfer/quant_spec.h"
#include "intfer/spinquant.hpp"

using namespace intfer;

extern "C" {

uint16_t ref_float_to_half(float v) { return dashq::float_to_half(v); }
float ref_half_to_float(uint16_t h) { return dashq::half_to_float(h); }

// GA=64 act-quant of one row of K floats; round 0 = HalfAway, 1 = RoundNear.
void ref_act_quant_ga64(const float* x, int8_t* q, float* scales, size_t K, int round) {
  dashq::act_quant_ga64_batch(x, q, scales, K,
                              round == 0 ? dashq::ActQuantRound::HalfAway
                                         : dashq::ActQuantRound::RoundNear);
}

void ref_act_quant_scale_inv(const float* x, size_t M, size_t K, float* out) {
  dashq::act_quant_ga64_scale_inv_batch(x, M, K, out);
}

int ref_avx2_available(void) { return dashq::avx2_available() ? 1 : 0; }

// out = x R for the canonical Hadamard of `dim` (fast path), and the dense
// matrix itself (dim*dim, may be NULL).
int ref_rotation_fwht(uint32_t dim, const float* x, float* out, float* mat) {
  Rotation R = make_hadamard(dim);
  if (!rotation_is_hadamard(R)) return -1;
  apply_rotation_fwht(R, x, out);
  if (mat) std::memcpy(mat, R.mat.data(), R.mat.size() * sizeof(float));
  return 0;
}

void ref_canonical_codebook(int bits, float* out) {
  QuantScheme s = bits == 2 ? QuantScheme::INT2 : bits == 4 ? QuantScheme::INT4 : QuantScheme::INT8;
  std::vector<float> cb = dashq::canonical_codebook(s);
  std::memcpy(out, cb.data(), cb.size() * sizeof(float));
}

// Reference dequant of a group-major packed tensor with one fp16 scale per
// K-group shared by all N rows (QuantResult::dequant).
void ref_dequant(int bits, uint32_t N, uint32_t K, uint16_t G, const uint8_t* codes,
                 size_t code_bytes, const uint16_t* scales, uint32_t n_groups, float* out) {
  dashq::QuantResult r;
  r.qcfg.scheme = bits == 2 ? QuantScheme::INT2 : bits == 4 ? QuantScheme::INT4 : QuantScheme::INT8;
  r.qcfg.group_size = G;
  r.codes.assign(codes, codes + code_bytes);
  r.scales.resize((size_t)n_groups * 2);
  for (uint32_t g = 0; g < n_groups; ++g) {
    r.scales[2 * g] = (uint8_t)(scales[g] & 0xFF);
    r.scales[2 * g + 1] = (uint8_t)(scales[g] >> 8);
  }
  std::vector<float> o;
  r.dequant(o, N, K);
  std::memcpy(out, o.data(), o.size() * sizeof(float));
}

// Read an INTFER1 image with the reference reader and write it back with the
// reference writer.  Returns -1 if the reader rejects the image; else 0 and a
// malloc'd copy of the re-serialized bytes (free with ref_free).
int ref_intfer_reserialize(const uint8_t* blob, size_t n, uint8_t** out, size_t* out_n) {
  ModelIR m;
  RotationSet rs;
  if (!deserialize_intfer(blob, n, m, rs)) return -1;
  std::vector<uint8_t> b = serialize_intfer(m, rs);
  *out = static_cast<uint8_t*>(std::malloc(b.size() ? b.size() : 1));
  std::memcpy(*out, b.data(), b.size());
  *out_n = b.size();
  return 0;
}

// Reference dequant_tensor of the tensor named `name`: writes N*K floats to
// out (capacity cap) and returns N*K, or -1 if unreadable / absent / too big.
long ref_intfer_dequant(const uint8_t* blob, size_t n, const char* name, float* out, size_t cap) {
  ModelIR m;
  RotationSet rs;
  if (!deserialize_intfer_borrowed(blob, n, m, rs)) return -1;
  for (const TensorIR& t : m.tensors) {
    if (t.name != name) continue;
    std::vector<float> o;
    dashq::dequant_tensor(m, t, o);
    if (o.size() > cap) return -1;
    std::memcpy(out, o.data(), o.size() * sizeof(float));
    return (long)o.size();
  }
  return -1;
}

// The reference's Hadamard shape check of rotation i (rotation_is_hadamard,
// spinquant.cpp:607-629): 1 / 0, or -1 if unreadable.
int ref_intfer_rotation_is_hadamard(const uint8_t* blob, size_t n, int i) {
  ModelIR m;
  RotationSet rs;
  if (!deserialize_intfer(blob, n, m, rs) || i < 0 || (size_t)i >= rs.rotations.size()) return -1;
  return rotation_is_hadamard(rs.rotations[i]) ? 1 : 0;
}

void ref_free(void* p) { std::free(p); }

}  // extern "C"
