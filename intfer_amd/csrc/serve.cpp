// The --serve JSON-lines loop over the continuous-batching scheduler
// (run_serve, examples/intfer_cli/main.cpp:9260-9377): requests arrive as
// one JSON object per input line, are admitted FIFO under the scheduler's
// live cap, and every scheduler iteration streams its tokens and finished
// requests as JSON lines.  Single-threaded, like the reference's dispatcher.
#include <poll.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "host_model.h"
#include "intfer_amd.h"
#include "json_read.h"

using ifrh::fail;
using ifrh::JNode;
using ifrh::JReader;

namespace {

// The prompt the reference serves when a line's prompt yields no tokens
// (main.cpp:9304-9305).
const int32_t kFallbackPrompt[5] = {760, 6511, 314, 9338, 369};

std::string jstr(const std::string& s) {
  std::string o = "\"";
  for (const char c : s) {
    const unsigned char u = (unsigned char)c;
    if (c == '"' || c == '\\') {
      o += '\\';
      o += c;
    } else if (c == '\n') {
      o += "\\n";
    } else if (c == '\r') {
      o += "\\r";
    } else if (c == '\t') {
      o += "\\t";
    } else if (u < 0x20) {
      char b[8];
      std::snprintf(b, sizeof(b), "\\u%04x", u);
      o += b;
    } else {
      o += c;
    }
  }
  return o + "\"";
}

bool write_all(int fd, const std::string& s) {
  size_t off = 0;
  while (off < s.size()) {
    const ssize_t n = ::write(fd, s.data() + off, s.size() - off);
    if (n < 0) {
      if (errno == EINTR) continue;
      return false;
    }
    off += (size_t)n;
  }
  return true;
}

// A number field as an integer (JSON integer, or a real truncated toward
// zero like the reference's atoi / atol of the value).
bool as_int(const JNode* n, int64_t* v) {
  if (!n) return false;
  if (n->kind == JNode::Int) {
    *v = n->i;
    return true;
  }
  if (n->kind == JNode::Real && std::isfinite(n->d) && std::fabs(n->d) < 9e18) {
    *v = (int64_t)n->d;
    return true;
  }
  return false;
}
double as_real(const JNode* n) {
  if (!n) return 0;
  return n->kind == JNode::Int ? (double)n->i : n->kind == JNode::Real ? n->d : 0;
}

struct Request {
  std::vector<int32_t> prompt;
  int max_new = 64;
  bool has_id = false;
  int64_t id = 0;
  ifr_sample_params sp{};
};

// Parse one request line (parse_serve_line, main.cpp:8595-8676, with token
// ids in place of the prompt text).  Returns "" or the refusal message.
std::string parse_line(const std::string& line, const ifr_serve_cfg& cfg, int32_t kv_cap,
                       Request& r) {
  JNode root;
  JReader rd(line.data(), line.data() + line.size());
  if (!rd.document(root) || root.kind != JNode::Obj) return "malformed request line";
  int64_t v = 0;
  if (as_int(root.at("id"), &v)) {
    r.id = v;
    r.has_id = true;
  }
  r.max_new = cfg.default_max_new > 0 ? cfg.default_max_new : 64;
  if (as_int(root.at("max_new"), &v)) r.max_new = (int)std::max<int64_t>(std::min<int64_t>(v, 1 << 30), -1);
  if (r.max_new < 1) r.max_new = 1;
  if (r.max_new > 4096) r.max_new = 4096;
  // sampling keys over the serve defaults; top_k >= 0, top_p in [0, 1]
  // (parse_serve_line, main.cpp:8646-8668)
  r.sp.temperature = cfg.temperature;
  r.sp.top_k = cfg.top_k;
  r.sp.top_p = cfg.top_p;
  if (const JNode* t = root.at("temperature")) r.sp.temperature = (float)as_real(t);
  if (as_int(root.at("top_k"), &v)) r.sp.top_k = (int32_t)std::max<int64_t>(std::min<int64_t>(v, INT32_MAX), 0);
  if (const JNode* t = root.at("top_p")) r.sp.top_p = (float)as_real(t);
  if (r.sp.top_k < 0) r.sp.top_k = 0;
  if (r.sp.top_p < 0.f) r.sp.top_p = 0.f;
  if (r.sp.top_p > 1.f) r.sp.top_p = 1.f;
  if (as_int(root.at("seed"), &v)) {
    r.sp.seed = (uint32_t)v;
    r.sp.has_seed = 1;
  }
  const JNode* ids = root.at("prompt_ids");
  if (!ids) {
    if (root.at("prompt")) return "text prompts need a tokenizer: send prompt_ids";
    return "malformed request line";
  }
  if (ids->kind != JNode::Arr) return "malformed request line";
  for (const JNode& t : ids->items) {
    if (t.kind != JNode::Int) return "malformed request line";
    if (t.i < 0 || (cfg.vocab > 0 && t.i >= cfg.vocab) || t.i > INT32_MAX) return "token id out of range";
    r.prompt.push_back((int32_t)t.i);
  }
  if (r.prompt.empty()) r.prompt.assign(kFallbackPrompt, kFallbackPrompt + 5);
  if (cfg.vocab > 0)
    for (int32_t t : r.prompt)
      if (t >= cfg.vocab) return "token id out of range";
  if ((int64_t)r.prompt.size() + r.max_new > kv_cap) {
    char b[128];
    std::snprintf(b, sizeof(b), "prompt + max_new exceed the KV capacity of %d tokens", kv_cap);
    return b;
  }
  return "";
}

int work_left(ifr_sched* s) {
  int32_t live = 0, pre = 0, pend = 0;
  ifr_sched_info(s, &live, &pre, &pend, nullptr);
  return live + pre + pend;
}

}  // namespace

extern "C" int ifr_serve(ifr_sched* s, int32_t in_fd, int32_t out_fd, const ifr_serve_cfg* cfgp) {
  if (!s || in_fd < 0 || out_fd < 0) return fail(IFR_EINVAL, "serve: bad argument");
  const ifr_serve_cfg cfg = cfgp ? *cfgp : ifr_serve_cfg{};
  int32_t kv_cap = 0;
  if (int r = ifr_sched_info(s, nullptr, nullptr, nullptr, &kv_cap)) return r;
  if (int r = ifr_sched_record_events(s, 1)) return r;
  std::map<int64_t, int64_t> client_of;  // scheduler id -> the line's id
  int64_t next_id = 1;
  std::string inbuf;
  bool eof = false;
  std::vector<ifr_sched_event> ev(512);
  int rc = IFR_OK;
  for (;;) {
    // Poll input without blocking while requests run; block while idle
    // (main.cpp:9312-9325, :9364-9372).
    if (!eof) {
      pollfd p{in_fd, POLLIN, 0};
      const int pr = ::poll(&p, 1, work_left(s) > 0 ? 0 : -1);
      if (pr < 0 && errno != EINTR) {
        eof = true;
      } else if (pr > 0) {
        char buf[1 << 16];
        const ssize_t n = ::read(in_fd, buf, sizeof(buf));
        if (n > 0) inbuf.append(buf, (size_t)n);
        else if (n == 0 || (errno != EINTR && errno != EAGAIN)) eof = true;
      }
    }
    std::string out;
    for (;;) {
      const size_t nl = inbuf.find('\n');
      if (nl == std::string::npos && !(eof && !inbuf.empty())) break;
      std::string line = inbuf.substr(0, nl == std::string::npos ? inbuf.size() : nl);
      inbuf.erase(0, nl == std::string::npos ? inbuf.size() : nl + 1);
      if (!line.empty() && line.back() == '\r') line.pop_back();
      if (line.find_first_not_of(" \t") == std::string::npos) continue;
      Request r;
      const std::string err = parse_line(line, cfg, kv_cap, r);
      if (!err.empty()) {
        out += "{" + (r.has_id ? "\"id\":" + std::to_string(r.id) + "," : std::string()) +
               "\"error\":" + jstr(err) + "}\n";
        continue;
      }
      if (!r.has_id) r.id = next_id++;
      else if (r.id >= next_id) next_id = r.id + 1;
      // a request without a seed draws from mt19937(seed + its id) (main.cpp:9305)
      if (!r.sp.has_seed) {
        r.sp.seed = cfg.seed + (uint32_t)r.id;
        r.sp.has_seed = 1;
      }
      int64_t sid = 0;
      if (ifr_sched_submit_sampled(s, r.prompt.data(), (int32_t)r.prompt.size(), r.max_new, &r.sp, &sid) !=
          IFR_OK) {
        out += "{\"id\":" + std::to_string(r.id) + ",\"error\":\"request refused by the scheduler\"}\n";
        continue;
      }
      client_of[sid] = r.id;
    }
    if (work_left(s) > 0) {
      int32_t nrun = 0;
      if (int e = ifr_sched_step(s, &nrun)) {
        out += "{\"error\":" + jstr(std::string("forward failed: ") + ifr_last_error()) + "}\n";
        write_all(out_fd, out);
        rc = e;
        break;
      }
      for (;;) {
        int32_t n = 0;
        ifr_sched_events(s, ev.data(), (int32_t)ev.size(), &n);
        for (int32_t i = 0; i < n; ++i) {
          const ifr_sched_event& e = ev[(size_t)i];
          const int64_t cid = client_of.count(e.id) ? client_of[e.id] : e.id;
          if (e.done) {
            out += "{\"id\":" + std::to_string(cid) + ",\"done\":true,\"generated\":" +
                   std::to_string(e.generated) + "}\n";
            client_of.erase(e.id);
            ifr_sched_release(s, e.id);
          } else {
            out += "{\"id\":" + std::to_string(cid) + ",\"token\":" + std::to_string(e.token) + "}\n";
          }
        }
        if (n < (int32_t)ev.size()) break;
      }
    }
    if (!out.empty() && !write_all(out_fd, out)) {
      rc = fail(IFR_EINVAL, "serve: output closed");
      break;
    }
    if (eof && inbuf.empty() && work_left(s) == 0) break;
  }
  ifr_sched_record_events(s, 0);
  return rc;
}
