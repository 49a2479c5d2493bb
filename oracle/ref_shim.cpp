// CPU ORACLE PIN -- test infrastructure only.
//
// extern "C" entry points over the reference's own host quant core, compiled
// from the sources where they lie under the reference root (see
// oracle/Makefile, target `ref`).  The output library lives in oracle/_ref/
// (git-ignored) and is used only by tests/ to pin the oracle restatement
// against the reference's code: fp16 conversion (src/quant/dashq.cpp:338-384),
// act-quant (dashq.cpp:221-336), the canonical codebook + dequant
// (dashq.cpp:405-417, :531-575) and the FWHT rotation (src/spinquant.cpp:99-125,
// :303-312, :586-629).
#include <cstdint>
#include <cstring>
#include <vector>

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

}  // extern "C"
