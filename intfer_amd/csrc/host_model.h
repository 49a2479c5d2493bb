// Library-owned host models (synthetic or parsed from an .intfer file): the
// buffers behind an ifr_host_model handed out through the C-ABI, released by
// ifr_host_model_free.
#pragma once
#include <cstdint>
#include <vector>

#include "intfer_amd.h"

namespace ifrh {

struct OwnedLinear {
  std::vector<uint8_t> codes;
  std::vector<uint16_t> scale, zero;
};

struct OwnedModel {
  ifr_host_model pub{};
  std::vector<float> embed, final_norm, lm_head;
  std::vector<ifr_layer_w> layers;
  std::vector<std::vector<float>> norms;  // 4 per layer: in_ln, post_ln, q_norm, k_norm
  std::vector<OwnedLinear> lin;           // 7 per layer: q, k, v, o, gate, up, down

  // Point pub's arrays at the owned buffers (after they are filled).
  void publish();
};

// Hand a model out: records it so ifr_host_model_free can release it.
ifr_host_model* adopt(OwnedModel* m);

// Record the message ifr_last_error() returns on this thread; returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace ifrh
