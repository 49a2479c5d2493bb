"""Sampling (S16) on the device engine: the scheduler's sampled streams are
the reference sampler (sample, main.cpp:8674-8764, restated in the CPU
oracle) applied to the device logits, with each request's own mt19937.

The expected stream of a request is rebuilt by driving the engine by hand,
one sequence alone: the prompt's last row gives the argmax (the first
token, main.cpp:8522-8523), then each decode row returns its logits (want =
2) and the oracle's sampler draws the token.  A row's result does not
depend on its batch, so the scheduler's batched run must match exactly.
A temperature near 0 reproduces the greedy stream."""
import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MAX_NEW = 12


def _replay(eng, prompt, seed, T, k, p):
    O = po.oracle()
    g = O.or_rng_create(seed)
    s = eng.seq_open()
    try:
        n = len(prompt)
        b = eng.forward([(s, i, t, ia.ROW_PREFILL, int(i == n - 1)) for i, t in enumerate(prompt)])
        out = [int(b[-1])]
        while len(out) < MAX_NEW + 1:
            _, lg = eng.forward([(s, n + len(out) - 1, out[-1], ia.ROW_DECODE, 2)], logits=True)
            out.append(O.or_sample(ptr(np.ascontiguousarray(lg[0])), lg.shape[1], k, p, T, g))
        return out
    finally:
        eng.seq_close(s)
        O.or_rng_free(g)


def test_sampled_streams_follow_the_reference_sampler(dev):
    cfg = ia.default_cfg(layers=2)
    m = ia.SynthModel(cfg, seed=11, bits=2)
    try:
        eng = ia.Engine(dev, m, max_seqs=16, max_seq_tokens=1024, max_rows=256)
        rng = np.random.default_rng(41)
        prompts = [rng.integers(0, cfg.vocab, size=int(n)).tolist() for n in (30, 75, 140, 52, 9)]
        params = [(0.8, 0, 0.0, None), (1.1, 40, 0.0, 123), (0.9, 0, 0.9, None), None, (1e-6, 0, 0.0, 5)]
        announce("sampled requests through the device scheduler")
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8, seed=2024)
        ids = []
        for pr, pa in zip(prompts, params):
            if pa is None:
                ids.append(sch.submit(pr, MAX_NEW))
            else:
                T, k, pp, sd = pa
                ids.append(sch.submit(pr, MAX_NEW, temperature=T, top_k=k, top_p=pp, seed=sd))
        for _ in range(500):
            if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                break
        got = [sch.result(i)[0] for i in ids]
        sch.close()
        greedy = {}
        for rid, pr, pa, g in zip(ids, prompts, params, got):
            assert len(g) == MAX_NEW + 1
            if pa is None:
                continue
            T, k, pp, sd = pa
            announce(f"replay of request {rid} (T={T}, top_k={k}, top_p={pp})")
            assert g == _replay(eng, pr, 2024 + rid if sd is None else sd, T, k, pp), rid
        # temperature -> 0: the greedy stream of the same prompt
        announce("greedy stream of the near-zero-temperature prompt")
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8)
        i0 = sch.submit(prompts[4], MAX_NEW)
        while not sch.result(i0)[1]:
            sch.step()
        assert sch.result(i0)[0] == got[4]
        sch.close()
    finally:
        m.close()
