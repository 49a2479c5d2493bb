"""Prefix reuse on the device engine.

  * ifr_seq_copy_prefix: a sequence built from a copied KV prefix plus the
    recomputed rest scores exactly (bit for bit) what the source sequence
    scored, with fp16 and int8 KV, at cuts inside and on page boundaries;
  * the scheduler's prefix cache (ifr_sched_cfg.prefix_cache, the
    reference's PrefixCache, examples/intfer_cli/main.cpp:9469-9720) streams
    the same tokens as the uncached scheduler on chat turns, where each
    prompt extends the previous exchange, and under concurrent load.
Exact equality holds because every kernel's result for a row is independent
of which other rows share its launch (fixed attention split, fixed GEMM
reduction order).
"""
import numpy as np
import pytest

import intfer_amd as ia
from tests.conftest import announce

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    cfg = ia.default_cfg(layers=4)
    m = ia.SynthModel(cfg, seed=13, bits=2)
    yield cfg, m
    m.close()


def _drive(sch, prompt, max_new):
    rid = sch.submit(prompt, max_new)
    for _ in range(2000):
        if sch.step() == 0 and sch.result(rid)[1]:
            break
    out, done = sch.result(rid)
    assert done
    return out


@pytest.mark.parametrize("kv8", [0, 1])
def test_copied_prefix_scores_bit_identically(dev, model, kv8):
    cfg, m = model
    eng = ia.Engine(dev, m, max_seqs=4, max_seq_tokens=1024, pool_tokens=4 * 1024, kv_int8=kv8,
                    max_rows=320)
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, cfg.vocab, size=300).tolist()
    a = eng.seq_open()
    announce(f"prefix copy kv_int8={kv8}: 300-token source")
    ba, la = eng.forward([(a, p, t, ia.ROW_PREFILL, int(p == 299)) for p, t in enumerate(prompt)],
                         logits=True)
    for cut in (1, 32, 200, 299):
        b = eng.seq_open()
        eng.seq_copy_prefix(b, a, cut)
        assert eng.seq_len(b) == cut
        _, lb = eng.forward([(b, p, prompt[p], ia.ROW_PREFILL, int(p == 299))
                             for p in range(cut, 300)], logits=True)
        assert np.array_equal(la, lb), (cut, float(np.abs(la - lb).max()))
        t = int(ba[-1])
        _, da = eng.forward([(a, 300, t, ia.ROW_DECODE, 1)], logits=True)
        _, db = eng.forward([(b, 300, t, ia.ROW_DECODE, 1)], logits=True)
        assert np.array_equal(da, db), cut
        eng.seq_truncate(a, 300)
        eng.seq_close(b)
    eng.seq_close(a)


def test_scheduler_cache_streams_equal_uncached(dev, model):
    cfg, m = model
    eng = ia.Engine(dev, m, max_seqs=24, max_seq_tokens=2048, max_rows=512)
    rng = np.random.default_rng(22)
    firsts = [rng.integers(0, cfg.vocab, size=int(n)).tolist() for n in (180, 64, 400)]
    outs = []
    for n in (0, 4):
        announce(f"scheduler prefix_cache={n}: chat turns and a concurrent wave")
        sch = ia.Scheduler(eng, chunk_m=128, live_cap=16, prefix_cache=n)
        got = []
        for p in firsts:               # turn 1, then turn 2 extending it
            g = _drive(sch, p, 6)
            got.append(g)
            got.append(_drive(sch, p + g + [5, 6, 7, 8], 6))
        # a wave sharing prefixes with the cached streams, all at once
        wave = [firsts[0][:150] + [9] * 20, firsts[1] + got[2][:3], firsts[2], firsts[0][:10]]
        ids = [sch.submit(p, 6) for p in wave]
        for _ in range(2000):
            if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                break
        got += [sch.result(i)[0] for i in ids]
        sch.close()
        outs.append(got)
    assert outs[0] == outs[1]
    assert all(len(g) == 7 for g in outs[0])
