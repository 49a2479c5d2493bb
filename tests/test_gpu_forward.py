"""Model-level parity of the device forward against the CPU oracle (a8 contract).

cfg1: one mixed iteration (4 decode rows at contexts 17/133/512/1000 with
seeded N(0,1) KV + one 60-row prefill chunk), full 0.8B-class model
(hidden 1024, 28 layers, 16q/8kv, hd 128, SwiGLU 3072, vocab 151936, INT2
G128).  Tolerance on logits: relative to the logit spread, stated below;
greedy tokens must match except at documented near-ties (oracle top-2
margin below the logit tolerance).
"""
import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from oracle import pyoracle as po
from tests.conftest import announce

pytestmark = pytest.mark.gpu

# |logit_gpu - logit_oracle| <= LOGIT_TOL * std(oracle logits of the row)
LOGIT_TOL = 0.02


@pytest.fixture(scope="module")
def model():
    cfg = ia.default_cfg()
    m = ia.SynthModel(cfg, seed=11, bits=2)
    yield m
    m.close()


def _setup(dev, model, kv_int8):
    cfg = model.cfg
    w = wl.cfg1(cfg, seed=1)
    eng = ia.Engine(dev, model, max_seqs=8, max_seq_tokens=2048, pool_tokens=8 * 2048,
                    kv_int8=kv_int8, max_rows=128)
    ora = po.OracleEngine(model, kv_int8=kv_int8, mode=0, max_seqs=8)
    dec_e, dec_o = [], []
    for (k, v) in w.kv:
        s = eng.seq_open()
        eng.load_kv(s, k, v)
        dec_e.append(s)
        so = ora.seq_open()
        kr = k.astype(np.float16).astype(np.float32)
        vr = v.astype(np.float16).astype(np.float32)
        if kv_int8:
            for arr in (kr, vr):
                flat = arr.reshape(-1, cfg.head_dim)
                for i in range(flat.shape[0]):
                    seg = np.ascontiguousarray(flat[i])
                    po.oracle().or_kv_int8_round(po.ptr(seg), cfg.head_dim)
                    flat[i] = seg
        ora.set_kv(so, kr.reshape(cfg.layers, k.shape[1], -1), vr.reshape(cfg.layers, k.shape[1], -1))
        dec_o.append(so)
    pe, pq = eng.seq_open(), ora.seq_open()
    return w, eng, ora, dec_e, dec_o, pe, pq


def _compare_logits(lg, lo, what):
    for r in range(lg.shape[0]):
        sd = lo[r].std()
        d = np.abs(lg[r] - lo[r]).max()
        assert d <= LOGIT_TOL * sd, f"{what} row {r}: max |dlogit| {d:.4g} > {LOGIT_TOL} * {sd:.4g}"


def _margin(lo, tok_a, tok_b):
    return abs(float(lo[tok_a]) - float(lo[tok_b]))


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_cfg1_mixed_iteration_and_greedy64(dev, model, kv_int8):
    w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, model, kv_int8)
    rows_e = wl.cfg1_rows(w, dec_e, pe)
    rows_o = wl.cfg1_rows(w, dec_o, pq)
    announce(f"cfg1 forward kv_int8={kv_int8} M={len(rows_e)}")
    be, lg = eng.forward(rows_e, logits=True)
    bo, lo = ora.forward(rows_o, logits=True)
    want = [i for i, r in enumerate(rows_e) if r[4]]
    assert len(want) == 5
    _compare_logits(lg, lo, "cfg1")
    for j, i in enumerate(want):
        if be[i] != bo[i]:
            assert _margin(lo[j], be[i], bo[i]) <= LOGIT_TOL * lo[j].std(), f"row {i}: token differs"
    # 64 greedy steps for the 5 sequences, each side feeding its own argmax
    seq_e = dec_e + [pe]
    seq_o = dec_o + [pq]
    pos = list(w.contexts) + [len(w.pre_tokens)]
    tok_e = [int(be[i]) for i in want]
    tok_o = [int(bo[i]) for i in want]
    stream_e, stream_o, ties = [list(tok_e)], [list(tok_o)], 0
    for step in range(64):
        announce(f"cfg1 greedy step {step} kv_int8={kv_int8}")
        re_ = [(s, p, t, 0, 1) for s, p, t in zip(seq_e, pos, tok_e)]
        ro_ = [(s, p, t, 0, 1) for s, p, t in zip(seq_o, pos, tok_o)]
        be2, lg2 = eng.forward(re_, logits=True)
        bo2, lo2 = ora.forward(ro_, logits=True)
        if tok_e == tok_o:
            _compare_logits(lg2, lo2, f"step {step}")
        for j in range(5):
            if be2[j] != bo2[j] and tok_e[j] == tok_o[j]:
                m = _margin(lo2[j], be2[j], bo2[j])
                assert m <= LOGIT_TOL * lo2[j].std(), f"step {step} seq {j}: divergence, margin {m}"
                ties += 1
        tok_e = [int(x) for x in be2]
        tok_o = [int(x) for x in bo2]
        stream_e.append(tok_e)
        stream_o.append(tok_o)
        pos = [p + 1 for p in pos]
    same = np.mean(np.array(stream_e) == np.array(stream_o))
    print(f"[cfg1 kv_int8={kv_int8}] greedy agreement {same:.4f}, documented near-ties {ties}")
    # non-degenerate stream: the model does not just repeat one token
    assert len(set(np.array(stream_e).reshape(-1).tolist())) > 50
    if ties == 0:
        assert stream_e == stream_o


def test_split_equals_joint_and_solo_equals_loaded(dev, model):
    """Serve split == joint (test_cpu_parity.sh:76-92) and solo == loaded
    (test_serve_load.sh:157-158), bit-exact token streams on the device."""
    eng = ia.Engine(dev, model, max_seqs=16, max_seq_tokens=1024, pool_tokens=16 * 1024,
                    max_rows=256)
    prompts = wl.cfg4_requests(6, seed=8, lo=40, hi=300)
    streams = []
    for split in (0, 1):
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8, split_iter=split)
        ids = [sch.submit(p, 12) for p in prompts]
        for _ in range(400):
            announce(f"sched split={split} step")
            if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                break
        streams.append([sch.result(i)[0] for i in ids])
        sch.close()
    assert streams[0] == streams[1]
    assert all(len(s) == 13 for s in streams[0])
    solo = ia.Scheduler(eng, chunk_m=64, live_cap=8)
    i0 = solo.submit(prompts[2], 12)
    while not solo.result(i0)[1]:
        solo.step()
    assert solo.result(i0)[0] == streams[0][2]
    solo.close()


def test_spec_verify_rows_keep_greedy_stream(dev, model):
    """n-gram verify rows (K=4) in the joint batch: greedy acceptance +
    KV rollback must give the same stream as plain decode."""
    eng = ia.Engine(dev, model, max_seqs=16, max_seq_tokens=1024, pool_tokens=16 * 1024,
                    max_rows=256)
    rng = np.random.default_rng(5)
    base = rng.integers(0, model.cfg.vocab, size=30).astype(np.int32)
    prompts = [np.concatenate([base, base, base[:7]]).astype(np.int32), base[:25].copy()]
    out = []
    for k in (0, 4):
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8, spec_k=k)
        ids = [sch.submit(p, 20) for p in prompts]
        n = 0
        while not all(sch.result(i)[1] for i in ids) and n < 200:
            announce(f"spec_k={k} step {n}")
            sch.step()
            n += 1
        out.append([sch.result(i)[0] for i in ids])
        sch.close()
    assert out[0] == out[1]
