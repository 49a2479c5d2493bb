"""cfg4 serve load on the full 28-layer 0.8B-class INT2 engine (the load
bench.py times): C in {4, 8, 32, 64} requests with prompts U[64, 2048], max_new 64,
greedy, chunk budget 512, round-robin prefill, live cap 64.

  * every request finishes with max_new + 1 generated tokens (the prefill's
    token plus max_new decode tokens, the reference's finish rule,
    main.cpp:8409-8410);
  * solo == loaded (scripts/gates/test_serve_load.sh:155-158): three
    requests (the first, the longest prompt, the shortest) run alone through
    a fresh scheduler give exactly their streams under the load.  A row's
    result does not depend on the rest of its batch (fixed attention split,
    row-independent kernels), so the streams must be identical.
"""
import time

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MAX_NEW = 64
CHUNK = 512
CAP = 2176  # prompts <= 2048 + 64 generated, rounded up to whole 32-token pages


@pytest.fixture(scope="module")
def engine(dev):
    cfg = ia.default_cfg()
    m = ia.SynthModel(cfg, seed=11, bits=2)
    eng = ia.Engine(dev, m, max_seqs=64, max_seq_tokens=CAP, pool_tokens=64 * CAP, max_rows=64 + CHUNK)
    yield cfg, eng
    del eng
    m.close()


def _run(eng, prompts):
    sch = ia.Scheduler(eng, chunk_m=CHUNK, live_cap=64)
    ids = [sch.submit(p, MAX_NEW) for p in prompts]
    iters = 0
    t0 = time.perf_counter()
    while True:
        n = sch.step()
        iters += 1
        if n == 0 and all(sch.result(i)[1] for i in ids):
            break
        assert iters < 20000, "load did not drain"
    dt = time.perf_counter() - t0
    res = [sch.result(i) for i in ids]
    sch.close()
    return res, iters, dt


@pytest.mark.parametrize("conc", [4, 8, 32, 64])
def test_cfg4_load_finishes_and_solo_equals_loaded(engine, conc):
    cfg, eng = engine
    prompts = wl.cfg4_requests(conc, seed=4, vocab=cfg.vocab)
    announce(f"cfg4 load C={conc}, 28 layers, max_new {MAX_NEW}, chunk {CHUNK}")
    loaded, iters, dt = _run(eng, prompts)
    print(f"[cfg4 C={conc}] {iters} iterations, {dt:.3f} s, {conc * MAX_NEW / dt:.0f} output tok/s")
    for i, (toks, done) in enumerate(loaded):
        assert done and len(toks) == MAX_NEW + 1, (i, done, len(toks))
        assert all(0 <= t < cfg.vocab for t in toks)
    lens = [len(p) for p in prompts]
    picks = sorted({0, int(np.argmax(lens)), int(np.argmin(lens))})
    for i in picks:
        announce(f"cfg4 C={conc} solo request {i} (prompt {lens[i]} tokens)")
        (solo,), _, _ = _run(eng, [prompts[i]])
        assert solo[1] and solo[0] == loaded[i][0], f"request {i}: solo stream differs from loaded"
