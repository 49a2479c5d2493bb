// Token sampling over one row of logits: the reference's `sample`
// (examples/intfer_cli/main.cpp:8674-8764), restated step for step so a
// request's stream matches the reference's for the same logits and seed.
//
//   temperature <= 0 is read as 1e-5                              (:8676)
//   p_i = expf((l_i - max) / T), normalised by their sequential sum  (:8730-8737)
//   top_k > 0 (and < vocab): zero every p below the k-th largest p,
//     renormalise                                                  (:8738-8744)
//   0 < top_p < 1: order tokens by p descending (std::sort with the same
//     comparator), keep the shortest prefix whose running sum reaches top_p,
//     zero the rest, renormalise                                   (:8745-8756)
//   r = U[0,1) from the request's mt19937; the first i whose running sum of p
//     reaches r, else the last token                               (:8757-8763)
//
// The draw r is std::uniform_real_distribution<float>(0, 1) of the
// reference's standard library (libstdc++'s generate_canonical<float, 24>
// over one 32-bit output x): r = float(x) * 2^-32, with r >= 1 replaced by
// the largest float below 1.  It is written out here so the stream does not
// depend on the library this file is built against.  The optional
// INTFER_SAMPLE_TOPK_DIRECT shortcut of the reference (:8695-8724) is a
// reformulation of the same result and is not reproduced.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <random>
#include <vector>

#include "intfer_amd.h"

namespace ifrh {
int fail(int code, const char* fmt, ...);
}

struct ifr_rng {
  std::mt19937 g;
};

namespace {

float uniform01(std::mt19937& g) {
  const uint32_t x = (uint32_t)g();
  const float r = std::ldexp((float)x, -32);  // float(x) rounds to nearest even; the scaling is exact
  return r >= 1.0f ? std::nextafter(1.0f, 0.0f) : r;
}

void normalise(std::vector<float>& p) {
  float sum = 0.f;
  for (float v : p) sum += v;
  for (float& v : p) v /= sum;
}

}  // namespace

extern "C" {

int ifr_rng_create(uint32_t seed, ifr_rng** out) {
  if (!out) return ifrh::fail(IFR_EINVAL, "rng: out is null");
  *out = new ifr_rng{std::mt19937(seed)};
  return IFR_OK;
}

void ifr_rng_free(ifr_rng* r) { delete r; }

int ifr_rng_uniform(ifr_rng* r, float* u) {
  if (!r || !u) return ifrh::fail(IFR_EINVAL, "rng: null argument");
  *u = uniform01(r->g);
  return IFR_OK;
}

int ifr_sample(const float* logits, int32_t vocab, int32_t top_k, float top_p, float temperature,
               ifr_rng* rng, int32_t* token) {
  if (!logits || !rng || !token || vocab <= 0) return ifrh::fail(IFR_EINVAL, "sample: bad argument");
  if (temperature <= 0.f) temperature = 1e-5f;
  const size_t V = (size_t)vocab;
  float mx = -1e30f;
  for (size_t i = 0; i < V; ++i)
    if (logits[i] > mx) mx = logits[i];
  std::vector<float> p(V);
  for (size_t i = 0; i < V; ++i) p[i] = std::exp((logits[i] - mx) / temperature);
  normalise(p);
  if (top_k > 0 && (size_t)top_k < V) {
    std::vector<float> s = p;
    std::nth_element(s.begin(), s.end() - top_k, s.end());
    const float kth = s[V - (size_t)top_k];
    for (float& v : p)
      if (v < kth) v = 0.f;
    normalise(p);
  }
  if (top_p > 0.f && top_p < 1.f) {
    std::vector<int> idx(V);
    for (size_t i = 0; i < V; ++i) idx[i] = (int)i;
    std::sort(idx.begin(), idx.end(), [&](int a, int b) { return p[(size_t)a] > p[(size_t)b]; });
    float cum = 0.f;
    size_t cut = V;
    for (size_t i = 0; i < V; ++i) {
      cum += p[(size_t)idx[i]];
      if (cum >= top_p) {
        cut = i + 1;
        break;
      }
    }
    for (size_t i = cut; i < V; ++i) p[(size_t)idx[i]] = 0.f;
    normalise(p);
  }
  const float r = uniform01(rng->g);
  float acc = 0.f;
  for (size_t i = 0; i < V; ++i) {
    acc += p[i];
    if (r <= acc) {
      *token = (int32_t)i;
      return IFR_OK;
    }
  }
  *token = (int32_t)(V - 1);
  return IFR_OK;
}

}  // extern "C"
