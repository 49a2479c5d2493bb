// Continuous-batching iteration scheduler over the C-ABI engine.
//
// Restates the reference serve loop's policy (examples/intfer_cli/main.cpp):
//   sched_iteration_joint :8427-8542  one forward = [decode rows of live
//                                     requests in live order | up to chunk_m
//                                     prefill rows of the prefill-queue head]
//   sched_iteration       :8382-8413  decode-only forward (split path)
//   serve_iteration       :9203-9259  joint, or split (chunk forward, then
//                                     decode forward) when split_iter is set
//   serve_rotate_unfilled :9187-9195  round-robin rotation of unfilled heads
//   run_serve admission   :9329-9342  FIFO admission while live < cap
//   finish rule           :8409-8410  EOS 248044/248046 or max_new+1 ids
// plus n-gram speculative verify rows (main.cpp:11522-11550 ngram_from,
// :11842-11931 verify / accept / rollback) as a third row kind: a speculating
// request contributes its token and K drafts as one causal verify group.
// Per-request sampling (sched_iteration_joint's qgreedy / sample choice,
// main.cpp:8505-8508): a non-greedy request's decode rows ask the forward for
// their logits (want = 2) and draw the token with ifr_sample.
#include <algorithm>
#include <deque>
#include <iterator>
#include <map>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "intfer_amd.h"

namespace ifrh {
// the library's error record (ifr_last_error): sets the message, returns code
int fail(int code, const char* fmt, ...);
}  // namespace ifrh

namespace {

using ifrh::fail;

constexpr int kEos0 = 248044, kEos1 = 248046;

// Adaptive draft width (SpecAdapt, main.cpp:11454-11511, restated without
// the second-device producer scores, which this path does not have): the
// width w in 1..cap maximising w * accept_ema / (w + 1), first maximum
// kept; the EMA moves a quarter of the way to each round's accepted /
// drafted ratio and stays inside [0.05, 0.95].  Scheduling only: it picks
// how many drafts a round verifies, never which tokens.
struct SpecAdapt {
  double accept_ema = 0.5;
  int choose(int cap) const {
    if (cap < 1) return 1;
    int best = 1;
    double best_score = -1.0;
    for (int w = 1; w <= cap; ++w) {
      const double score = ((double)w * accept_ema) / ((double)w + 1.0);
      if (score > best_score) {
        best_score = score;
        best = w;
      }
    }
    return best;
  }
  void observe(int accepted, int tried) {
    if (tried <= 0) return;
    const double r = (double)accepted / (double)tried;
    accept_ema = accept_ema * 0.75 + r * 0.25;
    if (accept_ema < 0.05) accept_ema = 0.05;
    if (accept_ema > 0.95) accept_ema = 0.95;
  }
};

struct Req {
  int64_t id = 0;
  std::vector<int32_t> prompt, generated;
  int token = -1, pos = 0, fill = 0, max_new = 0;
  bool finished = false;
  int slot = -1;
  // sampling (Request :4812-4815); greedy when all three are off (:8401)
  float temperature = 0.f, top_p = 0.f;
  int top_k = 0;
  ifr_rng* rng = nullptr;
  SpecAdapt adapt;  // this request's draft-width controller (spec_adapt)
  bool greedy() const { return temperature <= 0.f && top_k == 0 && top_p <= 0.f; }
  ~Req() { ifr_rng_free(rng); }
};

// Drafts: tokens following the last occurrence of `tok` in generated (stops
// at its end), else in the prompt continuing into generated (main.cpp:
// 11522-11550, restated exactly, including that a search hit at the end of
// `gen` yields nothing and ends the generated search).
std::vector<int32_t> ngram_from(const std::vector<int32_t>& gen, const std::vector<int32_t>& pr,
                                int tok, int K) {
  std::vector<int32_t> d;
  for (int occ = (int)gen.size() - 1; occ >= 0 && (int)d.size() < K; --occ) {
    if (gen[(size_t)occ] == tok) {
      for (int j = occ + 1; j < (int)gen.size() && (int)d.size() < K; ++j) d.push_back(gen[(size_t)j]);
      break;
    }
  }
  if ((int)d.size() < K) {
    for (int occ = (int)pr.size() - 1; occ >= 0 && (int)d.size() < K; --occ) {
      if (pr[(size_t)occ] == tok) {
        for (int j = occ + 1; j < (int)pr.size() && (int)d.size() < K; ++j) d.push_back(pr[(size_t)j]);
        for (int j = 0; j < (int)gen.size() && (int)d.size() < K; ++j) d.push_back(gen[(size_t)j]);
        break;
      }
    }
  }
  if ((int)d.size() > K) d.resize(K);
  return d;
}

bool is_eos(int t) { return t == kEos0 || t == kEos1; }


}  // namespace

// A finished request kept for prefix reuse (PrefixCache::Entry,
// main.cpp:9472-9493, the HTTP dispatcher's cache): its KV slot stays open
// and holds state_len positions of stream = prompt + generated (the last
// generated id was never forwarded, main.cpp:9540-9544).
struct CacheEntry {
  int slot;
  std::vector<int32_t> stream;
  int state_len;
};

struct ifr_sched {
  ifr_sched_backend be{};
  ifr_sched_cfg cfg{};
  int max_seq_tokens = 0;
  std::map<int64_t, std::unique_ptr<Req>> pool;
  std::deque<Req*> pending;
  std::vector<Req*> live;
  std::deque<Req*> prefill_q;
  int64_t next_id = 1;
  std::vector<ifr_row> last_rows;
  std::vector<ifr_row> rows;
  std::vector<int32_t> best;
  std::vector<float> logits;           // [rows with want = 2][vocab] of the last forward
  bool record = false;                 // ifr_sched_record_events
  std::deque<ifr_sched_event> events;
  std::deque<CacheEntry> cache;        // most recently used first

  bool caching() const { return cfg.prefix_cache > 0 && be.seq_copy_prefix; }

  // Draft width cap (main.cpp:11512-11514): spec_k, or 8 under spec_adapt
  // when spec_k is 0; 0 = no speculation.
  int spec_cap() const { return cfg.spec_adapt && cfg.spec_k < 1 ? 8 : cfg.spec_k; }

  // Drop the least recently used entry other than the one holding slot keep.
  bool evict_lru(int keep = -1) {
    for (auto it = cache.rbegin(); it != cache.rend(); ++it) {
      if (it->slot == keep) continue;
      be.seq_close(be.user, it->slot);
      cache.erase(std::next(it).base());
      return true;
    }
    return false;
  }

  // Retire a finished request: its slot becomes a cache entry
  // (PrefixCache::snapshot, main.cpp:9518-9546; only once the whole prompt
  // is in, main.cpp:9944-9945), or closes.
  void retire(Req* q) {
    if (q->slot < 0) return;
    if (caching() && !q->prompt.empty() && !q->generated.empty() &&
        q->fill == (int)q->prompt.size()) {
      CacheEntry e;
      e.slot = q->slot;
      e.stream = q->prompt;
      e.stream.insert(e.stream.end(), q->generated.begin(), q->generated.end());
      e.state_len = std::min((int)e.stream.size() - 1, q->pos);
      cache.push_front(std::move(e));
      while ((int)cache.size() > cfg.prefix_cache) evict_lru();
    } else {
      be.seq_close(be.user, q->slot);
    }
    q->slot = -1;
  }

  // Longest prefix of the prompt held by an entry (PrefixCache::match,
  // main.cpp:9603-9619; the most recently used entry wins ties), capped
  // below the whole prompt so the last prompt row still runs and scores the
  // first token (main.cpp:9874-9878).  Returns the length, *slot the entry's slot.
  int match(const Req& q, int* slot) const {
    int best = 0;
    *slot = -1;
    for (const CacheEntry& e : cache) {
      const size_t n = std::min({e.stream.size(), q.prompt.size(), (size_t)e.state_len});
      size_t h = 0;
      while (h < n && e.stream[h] == q.prompt[h]) ++h;
      if ((int)h > best) {
        best = (int)h;
        *slot = e.slot;
      }
    }
    if (best >= (int)q.prompt.size()) best = (int)q.prompt.size() - 1;
    return best;
  }

  // Admission of the pending head into a fresh slot, resuming from a cached
  // prefix where one matches (PrefixCache::install, main.cpp:9633-9716; the
  // call site main.cpp:9871-9886).  The copy covers the whole hit: the
  // reference resumes at the largest recurrent-state grid row <= hit, and
  // attention-only KV truncates anywhere.  Cache entries give way when slots
  // or pages run out; a copy that still cannot get pages prefills in full.
  bool admit(Req* q) {
    int src = -1;
    const int hit = caching() ? match(*q, &src) : 0;
    int32_t slot = -1;
    while (be.seq_open(be.user, &slot) != IFR_OK)
      if (!evict_lru(src)) return false;
    q->slot = slot;
    if (hit > 0) {
      int r;
      while ((r = be.seq_copy_prefix(be.user, slot, src, hit)) == IFR_ENOMEM)
        if (!evict_lru(src)) break;
      if (r == IFR_OK) {
        q->fill = hit;
        for (auto it = cache.begin(); it != cache.end(); ++it)
          if (it->slot == src) {
            CacheEntry e = std::move(*it);
            cache.erase(it);
            cache.push_front(std::move(e));
            break;
          }
      }
    }
    return true;
  }

  // A streamed token: where the reference's emit hook fires (decode rows in
  // live order, main.cpp:8405 / :8505; accepted drafts + correction of a
  // verify group).  The token that ends a prefill is not streamed.
  void emit(const Req& q, int32_t tok) {
    if (record) events.push_back({q.id, tok, 0, (int32_t)q.generated.size(), 0});
  }

  struct DecodeItem {
    Req* r;
    int row0;
    std::vector<int32_t> drafts;
    int lrow;  // its row among the want = 2 rows (sampling requests), else -1
  };

  int forward() {
    best.assign(rows.size(), -1);
    last_rows = rows;
    size_t nl = 0;
    for (const ifr_row& rw : rows) nl += rw.want == 2;
    if (nl) logits.resize(nl * (size_t)be.vocab);
    int r;
    // a refused forward (KV pages exhausted) changed nothing: cached
    // prefixes give their pages back first
    for (;;) {
      r = nl ? be.forward_logits(be.user, rows.data(), (int32_t)rows.size(), best.data(), logits.data())
             : be.forward(be.user, rows.data(), (int32_t)rows.size(), best.data());
      if (r != IFR_ENOMEM || !evict_lru()) break;
    }
    return r;
  }

  // Decode (or verify) rows for every live request (main.cpp:8438-8446).
  void build_decode(std::vector<DecodeItem>& items) {
    int nl = 0;
    for (Req* q : live) {
      if (q->finished) continue;
      if ((int)q->generated.size() >= q->max_new + 1) { q->finished = true; continue; }
      DecodeItem it{q, (int)rows.size(), {}, -1};
      if (!q->greedy()) {  // one decode row whose logits come back
        it.lrow = nl++;
        rows.push_back({q->slot, q->pos, q->token, IFR_ROW_DECODE, 2});
        items.push_back(std::move(it));
        continue;
      }
      if (spec_cap() > 0) {
        const int width = cfg.spec_adapt ? q->adapt.choose(spec_cap()) : cfg.spec_k;
        it.drafts = ngram_from(q->generated, q->prompt, q->token, width);
        while (!it.drafts.empty() && q->pos + (int)it.drafts.size() >= max_seq_tokens) it.drafts.pop_back();
      }
      const int kind = it.drafts.empty() ? IFR_ROW_DECODE : IFR_ROW_VERIFY;
      rows.push_back({q->slot, q->pos, q->token, kind, 1});
      for (size_t i = 0; i < it.drafts.size(); ++i)
        rows.push_back({q->slot, q->pos + 1 + (int)i, it.drafts[i], IFR_ROW_VERIFY, 1});
      items.push_back(std::move(it));
    }
  }

  // Advance decode / verify rows after the forward (main.cpp:8500-8515,
  // :11867-11931).
  int finish_decode(const std::vector<DecodeItem>& items) {
    for (const DecodeItem& it : items) {
      Req& q = *it.r;
      if (it.drafts.empty()) {
        int next = best[(size_t)it.row0];
        if (it.lrow >= 0) {
          if (int r = ifr_sample(logits.data() + (size_t)it.lrow * be.vocab, be.vocab, q.top_k, q.top_p,
                                 q.temperature, q.rng, &next))
            return r;
        }
        q.generated.push_back(next);
        q.pos++;
        emit(q, next);
        q.token = next;
        if (is_eos(next)) q.finished = true;
        if ((int)q.generated.size() >= q.max_new + 1) q.finished = true;
        continue;
      }
      const int K = (int)it.drafts.size();
      int a = 0;
      while (a < K && best[(size_t)it.row0 + a] == it.drafts[(size_t)a]) a++;
      if (cfg.spec_adapt) q.adapt.observe(a, K);
      const int corr = best[(size_t)it.row0 + a];
      std::vector<int32_t> acc;
      for (int i = 0; i < a; ++i) {
        acc.push_back(it.drafts[(size_t)i]);
        if (is_eos(it.drafts[(size_t)i])) break;
      }
      bool stopped = !acc.empty() && is_eos(acc.back());
      if (!stopped) acc.push_back(corr);
      int budget = q.max_new + 1 - (int)q.generated.size();
      if (budget < 1) budget = 1;
      while ((int)acc.size() > budget) acc.pop_back();
      stopped = !acc.empty() && is_eos(acc.back());
      const int n_draft_emit = (int)acc.size() - (stopped ? 0 : 1);
      const int pend = q.pos + n_draft_emit;
      if (int r = be.seq_truncate(be.user, q.slot, pend + 1)) return r;
      for (int t : acc) {
        q.generated.push_back(t);
        emit(q, t);
      }
      q.token = q.generated.back();
      q.pos = pend + 1;
      if (stopped) q.finished = true;
      if ((int)q.generated.size() >= q.max_new + 1) q.finished = true;
    }
    return IFR_OK;
  }

  void prefill_done(Req* pq, int best_id) {
    const int Sr = (int)pq->prompt.size();
    pq->generated.push_back(best_id);
    pq->token = best_id;
    pq->pos = Sr;
    live.push_back(pq);
  }

  // One chunk's prefill rows, appended to `rows`: the queue head's next
  // rows (main.cpp:8447-8470), or with pack_prefill the chunk budget filled
  // from the queue in order (a request whose prompt ends inside the chunk
  // leaves room for the next).  Returns the (request, rows) pieces.
  struct Piece {
    Req* q;
    int row0, n;
  };
  std::vector<Piece> build_prefill() {
    std::vector<Piece> pieces;
    int budget = cfg.chunk_m;
    for (Req* q : prefill_q) {
      if (budget == 0) break;
      const int Sr = (int)q->prompt.size();
      const int n = std::min(budget, Sr - q->fill);
      pieces.push_back({q, (int)rows.size(), n});
      for (int k = 0; k < n; ++k) {
        const int pos = q->fill + k;
        rows.push_back({q->slot, pos, q->prompt[(size_t)pos], IFR_ROW_PREFILL,
                        (q->fill + n == Sr && k == n - 1) ? 1 : 0});
      }
      budget -= n;
      if (!cfg.pack_prefill) break;
    }
    return pieces;
  }

  // After the forward: filled requests join live in queue order; an unfilled
  // head rotates to the back (serve_rotate_unfilled, main.cpp:9187-9195).
  void finish_prefill(const std::vector<Piece>& pieces) {
    for (const Piece& pc : pieces) {
      Req* q = pc.q;
      const int Sr = (int)q->prompt.size();
      q->fill += pc.n;
      if (q->fill == Sr) {
        prefill_q.erase(std::find(prefill_q.begin(), prefill_q.end(), q));
        prefill_done(q, best[(size_t)pc.row0 + pc.n - 1]);
      } else if (cfg.round_robin && prefill_q.size() > 1 && prefill_q.front() == q) {
        prefill_q.pop_front();
        prefill_q.push_back(q);
      }
    }
  }

  int joint(int32_t* nrun) {
    rows.clear();
    std::vector<DecodeItem> items;
    build_decode(items);
    const std::vector<Piece> pieces = build_prefill();
    *nrun = (int32_t)rows.size();
    if (rows.empty()) return IFR_OK;
    if (int r = forward()) return r;
    if (int r = finish_decode(items)) return r;
    finish_prefill(pieces);
    return IFR_OK;
  }

  int split(int32_t* nrun) {
    *nrun = 0;
    if (!prefill_q.empty()) {
      rows.clear();
      const std::vector<Piece> pieces = build_prefill();
      if (int r = forward()) return r;
      *nrun += (int32_t)rows.size();
      finish_prefill(pieces);
    }
    if (!live.empty()) {
      rows.clear();
      std::vector<DecodeItem> items;
      build_decode(items);
      if (!rows.empty()) {
        if (int r = forward()) return r;
        *nrun += (int32_t)rows.size();
        if (int r = finish_decode(items)) return r;
      }
    }
    return IFR_OK;
  }
};

extern "C" {

namespace {
int eng_open(void* u, int32_t* slot) { return ifr_seq_open(static_cast<ifr_ctx*>(u), slot); }
int eng_close(void* u, int32_t slot) { return ifr_seq_close(static_cast<ifr_ctx*>(u), slot); }
int eng_trunc(void* u, int32_t slot, int32_t len) {
  return ifr_seq_truncate(static_cast<ifr_ctx*>(u), slot, len);
}
int eng_fwd(void* u, const ifr_row* rows, int32_t M, int32_t* best) {
  return ifr_forward(static_cast<ifr_ctx*>(u), rows, M, best, nullptr);
}
int eng_fwd_logits(void* u, const ifr_row* rows, int32_t M, int32_t* best, float* logits) {
  return ifr_forward(static_cast<ifr_ctx*>(u), rows, M, best, logits);
}
int eng_copy(void* u, int32_t dst, int32_t src, int32_t len) {
  return ifr_seq_copy_prefix(static_cast<ifr_ctx*>(u), dst, src, len);
}
}  // namespace

int ifr_sched_create_backend(const ifr_sched_backend* be, const ifr_sched_cfg* cfg, ifr_sched** out) {
  if (!be || !cfg || !out || !be->seq_open || !be->seq_close || !be->seq_truncate || !be->forward)
    return fail(IFR_EINVAL, "sched: null argument or backend entry");
  if (cfg->chunk_m < 1 || cfg->chunk_m > 4096 || cfg->live_cap < 1 || cfg->spec_k < 0 ||
      cfg->spec_k > 15 || cfg->pack_prefill < 0 || cfg->pack_prefill > 1 || cfg->prefix_cache < 0 ||
      cfg->prefix_cache > 16 || cfg->spec_adapt < 0 || cfg->spec_adapt > 1 || be->kv_capacity <= 0 ||
      (be->forward_logits && be->vocab <= 0))
    return fail(IFR_EINVAL, "sched: configuration out of range");
  auto* s = new ifr_sched();
  s->be = *be;
  s->cfg = *cfg;
  s->max_seq_tokens = be->kv_capacity;
  *out = s;
  return IFR_OK;
}

int ifr_sched_create(ifr_ctx* ctx, const ifr_sched_cfg* cfg, ifr_sched** out) {
  if (!ctx) return fail(IFR_EINVAL, "sched: ctx is null");
  ifr_sched_backend be{};
  be.user = ctx;
  be.seq_open = eng_open;
  be.seq_close = eng_close;
  be.seq_truncate = eng_trunc;
  be.forward = eng_fwd;
  be.seq_copy_prefix = eng_copy;
  be.forward_logits = eng_fwd_logits;
  ifr_model_cfg mc{};
  if (int r = ifr_model_info(ctx, &mc)) return r;
  be.vocab = mc.vocab;
  if (int r = ifr_kv_capacity(ctx, &be.kv_capacity)) return r;
  return ifr_sched_create_backend(&be, cfg, out);
}

int ifr_sched_destroy(ifr_sched* s) {
  if (!s) return IFR_OK;
  for (auto& kv : s->pool)
    if (kv.second->slot >= 0) s->be.seq_close(s->be.user, kv.second->slot);
  for (const CacheEntry& e : s->cache) s->be.seq_close(s->be.user, e.slot);
  delete s;
  return IFR_OK;
}

int ifr_sched_submit(ifr_sched* s, const int32_t* prompt, int32_t n, int32_t max_new, int64_t* id) {
  return ifr_sched_submit_sampled(s, prompt, n, max_new, nullptr, id);
}

int ifr_sched_submit_sampled(ifr_sched* s, const int32_t* prompt, int32_t n, int32_t max_new,
                             const ifr_sample_params* sp, int64_t* id) {
  if (!s || !prompt || n <= 0 || max_new < 0)
    return fail(IFR_EINVAL, "sched_submit: null scheduler or prompt, n %d, max_new %d", n, max_new);
  auto r = std::make_unique<Req>();
  if (sp) {
    r->temperature = sp->temperature;
    r->top_k = sp->top_k < 0 ? 0 : sp->top_k;
    r->top_p = sp->top_p < 0.f ? 0.f : (sp->top_p > 1.f ? 1.f : sp->top_p);
  }
  r->id = s->next_id;
  if (!r->greedy()) {
    if (!s->be.forward_logits) return fail(IFR_EDECLINE, "sampling request needs a backend with forward_logits");
    // the request's generator (main.cpp:9305)
    if (int e = ifr_rng_create(sp->has_seed ? sp->seed : s->cfg.seed + (uint32_t)r->id, &r->rng)) return e;
  }
  s->next_id++;
  r->prompt.assign(prompt, prompt + n);
  r->max_new = max_new;
  if (id) *id = r->id;
  s->pending.push_back(r.get());
  s->pool[r->id] = std::move(r);
  return IFR_OK;
}

int ifr_sched_step(ifr_sched* s, int32_t* rows_run) {
  if (!s) return fail(IFR_EINVAL, "sched_step: scheduler is null");
  int32_t dummy = 0;
  if (!rows_run) rows_run = &dummy;
  *rows_run = 0;
  // admission: FIFO while live < cap and a KV slot is free
  while (!s->pending.empty() && (int)s->live.size() < s->cfg.live_cap) {
    Req* q = s->pending.front();
    if (!s->admit(q)) break;
    s->pending.pop_front();
    s->prefill_q.push_back(q);
  }
  int r = s->cfg.split_iter ? s->split(rows_run) : s->joint(rows_run);
  // A declined joint forward changed nothing: the same iteration runs the
  // split path, the chunk then the decode rows (serve_iteration,
  // main.cpp:9247-9256).
  if (r == IFR_EDECLINE && !s->cfg.split_iter) r = s->split(rows_run);
  if (r) return r;
  // live compaction; finished requests release their KV and report done
  // (run_serve's {"done"} accounting, main.cpp:9349-9363)
  std::vector<Req*> still;
  for (Req* q : s->live) {
    if (q->finished) {
      s->retire(q);
      if (s->record) s->events.push_back({q->id, -1, 1, (int32_t)q->generated.size(), 0});
    } else {
      still.push_back(q);
    }
  }
  s->live.swap(still);
  return IFR_OK;
}

int ifr_sched_result(ifr_sched* s, int64_t id, int32_t* out, int32_t cap, int32_t* n, int32_t* done) {
  if (!s) return fail(IFR_EINVAL, "sched_result: scheduler is null");
  auto it = s->pool.find(id);
  if (it == s->pool.end()) return fail(IFR_EINVAL, "sched_result: no request %lld", (long long)id);
  const Req& q = *it->second;
  const int k = std::min<int>(cap, (int)q.generated.size());
  for (int i = 0; i < k && out; ++i) out[i] = q.generated[(size_t)i];
  if (n) *n = (int32_t)q.generated.size();
  if (done) *done = q.finished ? 1 : 0;
  return IFR_OK;
}

int ifr_sched_record_events(ifr_sched* s, int32_t on) {
  if (!s) return fail(IFR_EINVAL, "sched_record_events: scheduler is null");
  s->record = on != 0;
  if (!s->record) s->events.clear();
  return IFR_OK;
}

int ifr_sched_events(ifr_sched* s, ifr_sched_event* out, int32_t cap, int32_t* n) {
  if (!s || (cap > 0 && !out) || !n) return fail(IFR_EINVAL, "sched_events: null argument");
  int32_t k = 0;
  while (k < cap && !s->events.empty()) {
    out[k++] = s->events.front();
    s->events.pop_front();
  }
  *n = k;
  return IFR_OK;
}

int ifr_sched_release(ifr_sched* s, int64_t id) {
  if (!s) return fail(IFR_EINVAL, "sched_release: scheduler is null");
  auto it = s->pool.find(id);
  if (it == s->pool.end()) return fail(IFR_EINVAL, "sched_release: no request %lld", (long long)id);
  if (!it->second->finished) return fail(IFR_ESTATE, "sched_release: request %lld not finished", (long long)id);
  s->pool.erase(it);
  return IFR_OK;
}

int ifr_sched_info(ifr_sched* s, int32_t* live, int32_t* prefill, int32_t* pending,
                   int32_t* kv_capacity) {
  if (!s) return fail(IFR_EINVAL, "sched_info: scheduler is null");
  if (live) *live = (int32_t)s->live.size();
  if (prefill) *prefill = (int32_t)s->prefill_q.size();
  if (pending) *pending = (int32_t)s->pending.size();
  if (kv_capacity) *kv_capacity = s->max_seq_tokens;
  return IFR_OK;
}

int ifr_sched_last_rows(ifr_sched* s, ifr_row* out, int32_t cap, int32_t* n) {
  if (!s) return fail(IFR_EINVAL, "sched_last_rows: scheduler is null");
  const int k = std::min<int>(cap, (int)s->last_rows.size());
  for (int i = 0; i < k && out; ++i) out[i] = s->last_rows[(size_t)i];
  if (n) *n = (int32_t)s->last_rows.size();
  return IFR_OK;
}

}  // extern "C"
