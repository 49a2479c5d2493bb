// intfer_serve: the --serve command line (examples/intfer_cli/main.cpp
// --serve, run_serve :9260-9377) over the MI355X engine.  Loads an .intfer
// model (-m) or a seeded synthetic one (--synth), then serves JSON request
// lines from stdin and streams JSON event lines to stdout (ifr_serve).
// The reference's scheduler environment knobs are honoured:
// INTFER_PREFILL_CHUNK_M, INTFER_SERVE_MAX, INTFER_SPLIT_ITER, INTFER_PREFILL_RR.
#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "intfer_amd.h"

namespace {

void usage() {
  std::fprintf(stderr,
               "usage: intfer_serve (-m MODEL.intfer | --synth SEED [--bits 2|4|0] [--intfer-form])\n"
               "  [--hidden H --layers L --heads NQ --kv-heads NKV --inter F --vocab V]\n"
               "  [--kv-int8] [--max-new N] [--chunk-m N] [--live-cap N] [--split-iter] [--no-rr]\n"
               "  [--spec-k K] [--pack-prefill] [--prefix-cache N] [--max-seq-tokens N] [--max-seqs N]\n"
               "  [--pool-tokens N] [--device D] [-t TEMP] [-k TOP_K] [-T TOP_P] [-S SEED]\n");
}

int env_int(const char* name, int dflt, int lo, int hi) {
  const char* v = std::getenv(name);
  if (!v) return dflt;
  const int x = std::atoi(v);
  return (x >= lo && x <= hi) ? x : dflt;
}

}  // namespace

int main(int argc, char** argv) {
  ifr_model_cfg cfg;
  ifr_default_cfg(&cfg);
  std::string model_path;
  long long synth_seed = -1;
  int bits = 2, intfer_form = 0, kv_int8 = 0, max_new = 64, spec_k = 0, device = 0;
  int chunk_m = env_int("INTFER_PREFILL_CHUNK_M", 128, 1, 1024);
  int live_cap = env_int("INTFER_SERVE_MAX", 64, 1, 64);
  int split_iter = std::getenv("INTFER_SPLIT_ITER") ? 1 : 0;
  int rr = (std::getenv("INTFER_PREFILL_RR") && std::string(std::getenv("INTFER_PREFILL_RR")) == "0") ? 0 : 1;
  int max_seq_tokens = 4096, max_seqs = 0, pack = 0, pcache = 0;
  long long pool_tokens = 0;
  float temperature = 0.f, top_p = 0.f;
  int top_k = 0;
  uint32_t seed = 0;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        usage();
        std::exit(2);
      }
      return argv[++i];
    };
    if (a == "-m") model_path = next();
    else if (a == "--synth") synth_seed = std::atoll(next());
    else if (a == "--bits") bits = std::atoi(next());
    else if (a == "--intfer-form") intfer_form = 1;
    else if (a == "--hidden") cfg.hidden = std::atoi(next());
    else if (a == "--layers") cfg.layers = std::atoi(next());
    else if (a == "--heads") cfg.n_heads = std::atoi(next());
    else if (a == "--kv-heads") cfg.n_kv = std::atoi(next());
    else if (a == "--inter") cfg.inter = std::atoi(next());
    else if (a == "--vocab") cfg.vocab = std::atoi(next());
    else if (a == "--kv-int8") kv_int8 = 1;
    else if (a == "--max-new") max_new = std::atoi(next());
    else if (a == "--chunk-m") chunk_m = std::atoi(next());
    else if (a == "--live-cap") live_cap = std::atoi(next());
    else if (a == "--split-iter") split_iter = 1;
    else if (a == "--no-rr") rr = 0;
    else if (a == "--spec-k") spec_k = std::atoi(next());
    else if (a == "--pack-prefill") pack = 1;
    else if (a == "--prefix-cache") pcache = std::atoi(next());
    else if (a == "--max-seq-tokens") max_seq_tokens = std::atoi(next());
    else if (a == "--max-seqs") max_seqs = std::atoi(next());
    else if (a == "--pool-tokens") pool_tokens = std::atoll(next());
    else if (a == "--device") device = std::atoi(next());
    else if (a == "-t") temperature = (float)std::atof(next());
    else if (a == "-k") top_k = std::atoi(next());
    else if (a == "-T") top_p = (float)std::atof(next());
    else if (a == "-S") seed = (uint32_t)std::atoi(next());
    else {
      usage();
      return 2;
    }
  }
  if (model_path.empty() == (synth_seed < 0)) {
    usage();
    return 2;
  }
  // cached prefixes hold a sequence slot each
  if (max_seqs <= 0) max_seqs = live_cap + 4 + pcache;
  if (pool_tokens <= 0) pool_tokens = (long long)max_seqs * max_seq_tokens;
  ifr_kv_cfg kv{};
  kv.max_seqs = max_seqs;
  kv.max_seq_tokens = max_seq_tokens;
  kv.pool_tokens = (int32_t)pool_tokens;
  kv.kv_int8 = kv_int8;
  kv.max_rows = live_cap * (1 + spec_k) + chunk_m;

  ifr_ctx* ctx = nullptr;
  if (ifr_ctx_create(device, &ctx) != IFR_OK) {
    std::fprintf(stderr, "FAIL: device %d: %s\n", device, ifr_last_error());
    return 1;
  }
  int rc;
  if (!model_path.empty()) {
    std::fprintf(stderr, "[intfer] serve: loading %s\n", model_path.c_str());
    rc = ifr_model_load_intfer_file(ctx, model_path.c_str(), &cfg, &kv);
  } else {
    std::fprintf(stderr, "[intfer] serve: synthetic model seed %lld bits %d\n", synth_seed, bits);
    ifr_host_model* m = ifr_synth_model(&cfg, (uint64_t)synth_seed, bits | (intfer_form ? IFR_SYNTH_INTFER : 0));
    rc = m ? ifr_model_load(ctx, m, &kv) : IFR_EINVAL;
    ifr_host_model_free(m);
  }
  if (rc != IFR_OK) {
    std::fprintf(stderr, "FAIL: model load: %s\n", ifr_last_error());
    ifr_ctx_destroy(ctx);
    return 1;
  }
  ifr_sched_cfg sc{};
  sc.chunk_m = chunk_m;
  sc.live_cap = live_cap;
  sc.split_iter = split_iter;
  sc.round_robin = rr;
  sc.spec_k = spec_k;
  sc.pack_prefill = pack;
  sc.prefix_cache = pcache;
  ifr_sched* s = nullptr;
  if (ifr_sched_create(ctx, &sc, &s) != IFR_OK) {
    std::fprintf(stderr, "FAIL: scheduler: %s\n", ifr_last_error());
    ifr_ctx_destroy(ctx);
    return 1;
  }
  std::fprintf(stderr,
               "[intfer] serve: live cap %d, chunk %d, %s, spec_k %d, KV %s, %d x %d tokens, prefix cache %d\n",
               live_cap, chunk_m, split_iter ? "split" : "joint", spec_k, kv_int8 ? "int8" : "fp16",
               max_seqs, max_seq_tokens, pcache);
  // the reference's sampling defaults (-t / -k / -T) and base seed (-S; 0
  // picks one from the clock, main.cpp:10590-10591, printed to reproduce)
  if (seed == 0) {
    seed = (uint32_t)std::chrono::high_resolution_clock::now().time_since_epoch().count();
    if (temperature > 0.f || top_k > 0 || top_p > 0.f) std::fprintf(stderr, "[intfer] serve: seed %u\n", seed);
  }
  ifr_serve_cfg scfg{};
  scfg.default_max_new = max_new;
  scfg.vocab = cfg.vocab;
  scfg.temperature = temperature;
  scfg.top_k = top_k;
  scfg.top_p = top_p;
  scfg.seed = seed;
  rc = ifr_serve(s, STDIN_FILENO, STDOUT_FILENO, &scfg);
  if (rc != IFR_OK) std::fprintf(stderr, "FAIL: serve: %s\n", ifr_last_error());
  ifr_sched_destroy(s);
  ifr_ctx_destroy(ctx);
  return rc == IFR_OK ? 0 : 1;
}
