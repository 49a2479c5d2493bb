"""Serve-load harness for the intfer_serve command line (cfg4).

Counterpart of the reference's serve load gate (scripts/gates/test_serve_load.sh):
at each concurrency level C, C requests are sent to one running server at
once and the client-observed completion latency of each is recorded.
Reported per level: wall time, req/s, output tok/s (generated tokens, as the
done lines count them), P50 / P99 completion latency and mean time to the
first streamed token.  Gates, as in the reference:
  1. every request at every level finishes;
  2. the first request streams the same tokens under the top level's load as
     it did alone (greedy determinism under continuous batching);
  3. the top level's tok/s is not below the first level's.
Requests follow cfg4: prompt lengths U[64, 2048] of uniform token ids
(seeded), max_new 64, greedy.  The server speaks the JSON-lines protocol of
ifr_serve ({"prompt_ids":[...],"max_new":N,"id":K} in; token / done lines out).

    python -m intfer_amd.serve_load --synth 11 --levels 1 4 8 32 64 -- --chunk-m 512

Arguments after `--` go to intfer_serve unchanged.
"""
from __future__ import annotations

import argparse
import json
import queue
import subprocess
import sys
import threading
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BIN = HERE / "intfer_serve"


def pct(xs, p):
    if not xs:
        return float("nan")
    s = sorted(xs)
    k = (len(s) - 1) * p / 100.0
    f, c = int(k), min(int(k) + 1, len(s) - 1)
    return s[f] + (s[c] - s[f]) * (k - f)


def cfg4_prompts(n, seed=4, vocab=151936, lo=64, hi=2048):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n)
    return [rng.integers(0, vocab, size=int(k)).tolist() for k in lens]


class Server:
    """One intfer_serve process; events are read on a thread with arrival times."""

    def __init__(self, args, log_path=None):
        self.log = open(log_path, "w") if log_path else subprocess.DEVNULL
        self.p = subprocess.Popen([str(BIN), *args], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                  stderr=self.log, bufsize=0)
        self.q: queue.Queue = queue.Queue()
        self.t = threading.Thread(target=self._read, daemon=True)
        self.t.start()

    def _read(self):
        for raw in self.p.stdout:
            self.q.put((time.perf_counter(), json.loads(raw)))
        self.q.put((time.perf_counter(), None))

    def send(self, lines):
        self.p.stdin.write("".join(ln + "\n" for ln in lines).encode())
        self.p.stdin.flush()

    def close(self, timeout=120):
        try:
            self.p.stdin.close()
        except OSError:
            pass
        rc = self.p.wait(timeout=timeout)
        if self.log is not subprocess.DEVNULL:
            self.log.close()
        return rc


def run_level(srv: Server, prompts, ids, max_new, timeout):
    """Send one request per prompt at once; wait until all are done."""
    t0 = time.perf_counter()
    srv.send([json.dumps({"prompt_ids": p, "max_new": max_new, "id": i}) for p, i in zip(prompts, ids)])
    want = set(ids)
    toks = {i: [] for i in ids}
    first, done_t, gen = {}, {}, {}
    while want - set(done_t):
        try:
            t, ev = srv.q.get(timeout=timeout)
        except queue.Empty:
            raise RuntimeError(f"no server output for {timeout}s; "
                               f"{len(want) - len(done_t)} requests unfinished")
        if ev is None:
            raise RuntimeError("server exited before every request finished")
        if "error" in ev:
            raise RuntimeError(f"server error: {ev}")
        i = ev.get("id")
        if i not in want:
            continue
        if "token" in ev:
            toks[i].append(ev["token"])
            first.setdefault(i, t)
        elif ev.get("done"):
            done_t[i] = t
            gen[i] = ev["generated"]
    wall = time.perf_counter() - t0
    lat = [done_t[i] - t0 for i in ids]
    ttft = [first[i] - t0 for i in ids if i in first]
    ctoks = sum(gen.values())
    return dict(C=len(ids), wall_s=wall, req_s=len(ids) / wall, tok_s=ctoks / wall,
                lat_p50_s=pct(lat, 50), lat_p99_s=pct(lat, 99),
                ttft_mean_s=float(np.mean(ttft)) if ttft else float("nan"), ctoks=ctoks,
                all_done=all(gen[i] == max_new + 1 for i in ids)), toks


def sweep(server_args, levels, max_new=64, seed=4, vocab=151936, timeout=600, log_path=None,
          out=sys.stdout):
    prompts = cfg4_prompts(max(levels), seed=seed, vocab=vocab)
    srv = Server(server_args, log_path)
    results, fails = [], []
    solo, solo_stream = None, []
    next_id = 1
    try:
        solo, solo_toks = run_level(srv, prompts[:1], [next_id], max_new, timeout)
        solo_stream = solo_toks[next_id]
        next_id += 1
        for C in levels:
            ids = list(range(next_id, next_id + C))
            next_id += C
            r, toks = run_level(srv, prompts[:C], ids, max_new, timeout)
            results.append(r)
            print(f"c{C}: wall={r['wall_s']:.2f}s req/s={r['req_s']:.2f} tok/s={r['tok_s']:.1f} "
                  f"lat_p50={r['lat_p50_s']:.2f}s lat_p99={r['lat_p99_s']:.2f}s "
                  f"ttft_mean={r['ttft_mean_s']:.2f}s ctoks={r['ctoks']}", file=out, flush=True)
            if not r["all_done"]:
                fails.append(f"c{C}.all")
            if C == levels[-1]:
                r["parity"] = toks[ids[0]] == solo_stream
                if not r["parity"]:
                    fails.append(f"c{C}.parity")
    finally:
        rc = srv.close()
    if rc != 0:
        fails.append(f"server exit {rc}")
    if len(results) > 1 and results[-1]["tok_s"] < results[0]["tok_s"]:
        fails.append("scaling")
    return dict(levels=results, solo=solo, solo_stream=solo_stream, fails=fails)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("-m", dest="model", help=".intfer model file")
    src.add_argument("--synth", type=int, help="synthetic model seed")
    ap.add_argument("--levels", type=int, nargs="+", default=[1, 4, 8, 32, 64])
    ap.add_argument("--max-new", type=int, default=64)
    ap.add_argument("--seed", type=int, default=4)
    ap.add_argument("--vocab", type=int, default=151936)
    ap.add_argument("--timeout", type=float, default=600)
    ap.add_argument("--log", default=None, help="server stderr log file")
    ap.add_argument("--json", default=None, help="write the results here")
    ap.add_argument("rest", nargs="*", help="arguments for intfer_serve (after --)")
    a = ap.parse_args(argv)
    server_args = (["-m", a.model] if a.model else ["--synth", str(a.synth)]) + a.rest
    res = sweep(server_args, a.levels, a.max_new, a.seed, a.vocab, a.timeout, a.log)
    for f in res["fails"]:
        print(f"FAIL {f}")
    if a.json:
        Path(a.json).write_text(json.dumps(res, indent=1))
    print("SERVE-LOAD:", "FAIL" if res["fails"] else "PASS", flush=True)
    return 1 if res["fails"] else 0


if __name__ == "__main__":
    sys.exit(main())
