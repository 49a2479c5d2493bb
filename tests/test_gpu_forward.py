"""Model-level parity of the device forward against the CPU oracle (a8 contract).

cfg1: one mixed iteration (4 decode rows at contexts 17/133/512/1000 with
seeded N(0,1) KV + one 60-row prefill chunk).  Every kernel is bit-exact
against the oracle except attention (fp32-accurate, not bit-identical), so:
  * a 1-layer model gives the same tokens and logits within 2e-3 sigma (most
    rows bit-identical; a rare int8 activation-code flip moves the rest);
  * the full 28-layer model drifts by such code flips, amplified layer by
    layer.  The bounds come from the noise floor of the contract, measured on
    the CPU alone (tests/floor/make_floor.py -> parity_floor_cfg1.json): the
    oracle's own forward run with two faithful fp32 attention orders (the
    reference's host loop and the device's 256-token split decomposition)
    on this workload.  Whatever separates those two is what no fp32
    attention can promise, so the device is held to K_FLOOR = 1.5 times the
    floor (one more sample of the same process): per logit row rms and max
    |d| / sigma and 1 - corr (sigma = the oracle row's std), the mean rms over
    all compared rows, and the tie margin below;
  * greedy decode runs 64 steps free-running, each side feeding its own
    argmax (the reference's token KATs, scripts/gates/test_cpu_parity.sh:
    53-63).  A sequence's streams must stay identical until a step where the
    two argmaxes differ, and every such divergence must be a near-tie: the
    oracle's margin between its token and the device's token below K_FLOOR
    times the largest margin at which the two oracle orders diverge.  The
    same 64 steps then run teacher-forced (both sides fed the oracle's
    token), so every step compares the same distribution: each disagreement
    there must be a tie by the same rule, and the agreement rate is reported;
  * the random-init model's logits are nearly flat (median top-2 margin 0.15
    sigma, so divergences within a few steps are expected of any fp32
    order).  Its large-margin variant (workloads.successor_model: the same
    layers, embedding N(0, 1) and an untied lm_head of permuted embedding
    rows, top-2 margins 2.3 - 5.1 sigma against a floor of at most 0.9 sigma)
    must give identical free-running 64-step streams on every sequence.
  Measured figures are printed, and written as JSON to $IFR_PARITY_OUT when
  that directory is set.
"""
import ctypes as C
import json
import os
from pathlib import Path

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from oracle import pyoracle as po
from tests.conftest import announce

pytestmark = pytest.mark.gpu

# The noise floor of the cfg1 contract (two faithful fp32 attention orders of
# the oracle against each other, CPU only; tests/floor/make_floor.py) and the
# factor the device may exceed it by.
FLOOR = json.loads((Path(__file__).resolve().parent / "floor" / "parity_floor_cfg1.json").read_text())
K_FLOOR = 1.5


def floor_bounds(kv_int8):
    f = FLOOR[f"kv{kv_int8}"]
    return {"rms": K_FLOOR * f["rms_sigma_max"], "max": K_FLOOR * f["max_sigma_max"],
            "corr": 1.0 - K_FLOOR * (1.0 - f["corr_min"]), "rms_mean": K_FLOOR * f["rms_sigma_mean"],
            "tie": K_FLOOR * f["divergence_margin_max"]}


# per-row bounds of every model-level comparison in this file and the tests
# that share _check_logits: the looser of the two KV formats' floors
_B = [floor_bounds(0), floor_bounds(1)]
RMS_TOL = max(b["rms"] for b in _B)
MAX_TOL = max(b["max"] for b in _B)
CORR_MIN = min(b["corr"] for b in _B)


@pytest.fixture(scope="module")
def model():
    cfg = ia.default_cfg()
    m = ia.SynthModel(cfg, seed=11, bits=2)
    yield m
    m.close()


def _setup(dev, model, kv_int8, intfer=None):
    cfg = model.cfg
    w = wl.cfg1(cfg, seed=1)
    eng = ia.Engine(dev, model if intfer is None else cfg, max_seqs=8, max_seq_tokens=2048,
                    pool_tokens=8 * 2048, kv_int8=kv_int8, max_rows=128, intfer=intfer)
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


def _check_logits(lg, lo, what, stats=None, bounds=None):
    rt, mt, cm = (RMS_TOL, MAX_TOL, CORR_MIN) if bounds is None else (bounds["rms"], bounds["max"], bounds["corr"])
    for r in range(lg.shape[0]):
        sd = float(lo[r].std())
        d = lg[r].astype(np.float64) - lo[r]
        rms = float(np.sqrt((d * d).mean()))
        corr = float(np.corrcoef(lg[r], lo[r])[0, 1])
        dmax = float(np.abs(d).max())
        if stats is not None:
            stats.append(rms / sd)
        assert rms <= rt * sd and corr >= cm and dmax <= mt * sd, (
            f"{what} row {r}: rms {rms:.4g} (tol {rt * sd:.4g}), corr {corr:.6f} (min {cm:.6f}), "
            f"max {dmax:.4g} (tol {mt * sd:.4g})")


def test_one_layer_bit_exact(dev):
    cfg = ia.default_cfg(layers=1)
    m = ia.SynthModel(cfg, seed=11, bits=2)
    try:
        w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, m, 0)
        announce("cfg1 one-layer bit-exact forward")
        be, lg = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
        bo, lo = ora.forward(wl.cfg1_rows(w, dec_o, pq), logits=True)
        assert np.array_equal(be, bo)
        exact = sum(np.array_equal(lg[r].view(np.uint32), lo[r].view(np.uint32)) for r in range(5))
        dmax = float(np.abs(lg - lo).max())
        print(f"[one layer] bit-identical logit rows {exact}/5, max |dlogit| {dmax:.3g}")
        assert exact >= 3 and dmax <= 2e-3 * float(lo.std())
    finally:
        m.close()


@pytest.mark.parametrize("intfer_form,bits", [(True, 0), (False, 2)])
def test_single_token_sequences_bit_exact(dev, intfer_form, bits):
    """Sequences of one token: attention over a single key is exact (softmax
    weight 1), so every kernel of the forward is bit-exact against the oracle
    and the whole logit rows must be too, up to a rare fp16 ulp of the device
    expf in SwiGLU.  The container form (post = 2/C, mixed INT2 / INT4 widths,
    so unfused QKV launches) runs through the same bar as the default form."""
    cfg = ia.default_cfg(layers=2)
    m = ia.SynthModel(cfg, seed=12, bits=bits, intfer_form=intfer_form)
    try:
        eng = ia.Engine(dev, m, max_seqs=16, max_seq_tokens=64, max_rows=64)
        ora = po.OracleEngine(m, kv_int8=0, mode=0, max_seqs=16)
        se = [eng.seq_open() for _ in range(12)]
        so = [ora.seq_open() for _ in range(12)]
        toks = [5 + 9973 * i for i in range(12)]
        announce(f"single-token sequences intfer_form={intfer_form} bits={bits}")
        be, lg = eng.forward([(s, 0, t, ia.ROW_DECODE, 1) for s, t in zip(se, toks)], logits=True)
        bo, lo = ora.forward([(s, 0, t, ia.ROW_DECODE, 1) for s, t in zip(so, toks)], logits=True)
        exact = sum(np.array_equal(lg[r].view(np.uint32), lo[r].view(np.uint32)) for r in range(12))
        print(f"[single token] form={intfer_form} bits={bits}: bit-identical rows {exact}/12, "
              f"max |dlogit| {float(np.abs(lg - lo).max()):.3g}")
        assert np.array_equal(be, bo) and exact >= 10
    finally:
        m.close()


def test_intfer_file_load_one_layer(dev, tmp_path):
    """A model loaded from its .intfer file (the mmap entry point) runs
    bit-identically to the host model it was written from.  Against the
    oracle on cfg1 (attention fp32-accurate, not bit-identical) it meets the
    model-level bounds of _check_logits and gives the same tokens: int8
    activation code flips move a few rows by up to ~0.06 sigma on this
    model, which the single-token test above shows is not the weights' form
    (there every row is bit-exact)."""
    cfg = ia.default_cfg(layers=1)
    m = ia.SynthModel(cfg, seed=12, bits=0, intfer_form=True)
    path = tmp_path / "one_layer.intfer"
    path.write_bytes(m.write_intfer("one-layer"))
    try:
        w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, m, 0)
        announce("intfer-form one-layer forward from the host model")
        be, lg = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
        bo, lo = ora.forward(wl.cfg1_rows(w, dec_o, pq), logits=True)
        del eng, ora
        w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, m, 0, intfer=path)
        announce("intfer-form one-layer forward from the .intfer file")
        bf, lf = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
        assert np.array_equal(bf, be)
        assert np.array_equal(lf.view(np.uint32), lg.view(np.uint32))
        assert np.array_equal(be, bo)
        exact = sum(np.array_equal(lg[r].view(np.uint32), lo[r].view(np.uint32)) for r in range(5))
        dmax = float(np.abs(lg - lo).max())
        print(f"[intfer one layer] bit-identical logit rows {exact}/5, max |dlogit| {dmax:.3g}")
        _check_logits(lg, lo, "intfer one layer")
    finally:
        m.close()


def _row_err(lg, lo):
    """(rms / sigma, max / sigma, corr) of one logit row against the oracle's."""
    sd = float(lo.std())
    d = lg.astype(np.float64) - lo
    return (float(np.sqrt((d * d).mean())) / sd, float(np.abs(d).max()) / sd,
            float(np.corrcoef(lg, lo)[0, 1]))


def _tie(lg, lo, t_e, t_o):
    """The divergence record of one row where the device chose t_e and the
    oracle t_o: the oracle's margin lo[t_o] - lo[t_e] and the device's
    lg[t_e] - lg[t_o], with the two tokens' logit errors, all in sigma."""
    sd = float(lo.std())
    return {"oracle_margin": float(lo[t_o] - lo[t_e]) / sd, "device_margin": float(lg[t_e] - lg[t_o]) / sd,
            "err_dev_token": float(lg[t_e] - lo[t_e]) / sd, "err_oracle_token": float(lg[t_o] - lo[t_o]) / sd,
            "token_device": int(t_e), "token_oracle": int(t_o)}


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_cfg1_mixed_iteration_and_greedy64(dev, model, kv_int8):
    fb = floor_bounds(kv_int8)
    w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, model, kv_int8)
    rows_e = wl.cfg1_rows(w, dec_e, pe)
    rows_o = wl.cfg1_rows(w, dec_o, pq)
    announce(f"cfg1 forward kv_int8={kv_int8} M={len(rows_e)}")
    be, lg = eng.forward(rows_e, logits=True)
    bo, lo = ora.forward(rows_o, logits=True)
    want = [i for i, r in enumerate(rows_e) if r[4]]
    assert len(want) == 5
    stats = []
    _check_logits(lg, lo, "cfg1", stats, fb)
    rec = {"kv_int8": kv_int8, "bounds": fb, "cfg1_tokens_equal": int(sum(be[i] == bo[i] for i in want)),
           "cfg1_row_err": [_row_err(lg[j], lo[j]) for j in range(5)], "ties": []}
    for j, i in enumerate(want):
        if be[i] != bo[i]:
            rec["ties"].append({"phase": "cfg1", "step": -1, "seq": j, **_tie(lg[j], lo[j], be[i], bo[i])})
    seq_e, seq_o = dec_e + [pe], dec_o + [pq]
    pos0 = [n + 1 for n in w.contexts] + [len(w.pre_tokens)]
    tok_e0 = [int(be[i]) for i in want]
    tok_o0 = [int(bo[i]) for i in want]
    errs = []
    # (1) free-running: each side feeds its own argmax; a sequence is compared
    # while its two streams are identical, and its first divergence must be a tie
    synced = [a == b for a, b in zip(tok_e0, tok_o0)]
    matched = [0 if not s else 64 for s in synced]
    tok_e, tok_o, pos = list(tok_e0), list(tok_o0), list(pos0)
    for step in range(64):
        announce(f"cfg1 free-running step {step} kv_int8={kv_int8}")
        b_e, l_e = eng.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_e, pos, tok_e)], logits=True)
        b_o, l_o = ora.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_o, pos, tok_o)], logits=True)
        for j in range(5):
            if not synced[j]:
                continue
            errs.append(_row_err(l_e[j], l_o[j]))
            _check_logits(l_e[j:j + 1], l_o[j:j + 1], f"free step {step} seq {j}", stats, fb)
            if b_e[j] != b_o[j]:
                rec["ties"].append({"phase": "free", "step": step, "seq": j,
                                    **_tie(l_e[j], l_o[j], b_e[j], b_o[j])})
                synced[j] = False
                matched[j] = step
        tok_e, tok_o = [int(x) for x in b_e], [int(x) for x in b_o]
        pos = [p + 1 for p in pos]
    rec["free_steps_identical"] = matched
    # (2) the same 64 steps teacher-forced from the cfg1 iteration's state
    for s, n in zip(seq_e, pos0):
        eng.seq_truncate(s, n)
    for s, n in zip(seq_o, pos0):
        ora.seq_truncate(s, n)
    tok, pos, agree, stream = list(tok_o0), list(pos0), 0, [list(tok_o0)]
    for step in range(64):
        announce(f"cfg1 teacher-forced step {step} kv_int8={kv_int8}")
        b_e, l_e = eng.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_e, pos, tok)], logits=True)
        b_o, l_o = ora.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_o, pos, tok)], logits=True)
        _check_logits(l_e, l_o, f"teacher-forced step {step}", stats, fb)
        for j in range(5):
            errs.append(_row_err(l_e[j], l_o[j]))
            if b_e[j] == b_o[j]:
                agree += 1
            else:
                rec["ties"].append({"phase": "forced", "step": step, "seq": j,
                                    **_tie(l_e[j], l_o[j], b_e[j], b_o[j])})
        tok = [int(x) for x in b_o]
        stream.append(tok)
        pos = [p + 1 for p in pos]
    e = np.array(errs)
    rec.update({"forced_agree": agree, "forced_rows": 320,
                "rms_sigma_mean": float(e[:, 0].mean()), "rms_sigma_max": float(e[:, 0].max()),
                "max_sigma_max": float(e[:, 1].max()), "corr_min": float(e[:, 2].min())})
    print(f"[cfg1 kv_int8={kv_int8}] free-running steps identical per sequence {matched}; "
          f"teacher-forced argmax agreement {agree}/320; logit rms/sigma mean {rec['rms_sigma_mean']:.4f} "
          f"max {rec['rms_sigma_max']:.4f}, max|d|/sigma {rec['max_sigma_max']:.4f}, corr min {rec['corr_min']:.5f}")
    for t in rec["ties"]:
        print(f"  tie {t['phase']} step {t['step']} seq {t['seq']}: oracle margin {t['oracle_margin']:.4f} sigma, "
              f"device margin {t['device_margin']:.4f}, token errors {t['err_dev_token']:+.4f} / "
              f"{t['err_oracle_token']:+.4f}")
    out = os.environ.get("IFR_PARITY_OUT")
    if out:
        os.makedirs(out, exist_ok=True)
        with open(os.path.join(out, f"parity_cfg1_kv{kv_int8}.json"), "w") as f:
            json.dump(rec, f, indent=1)
    # every divergence, free-running or forced, is a near-tie by the floor
    for t in rec["ties"]:
        assert 0 <= t["oracle_margin"] < fb["tie"], t
    # and on average the device sits at the floor, not just under its worst row
    assert rec["rms_sigma_mean"] <= fb["rms_mean"], (rec["rms_sigma_mean"], fb["rms_mean"])
    # a non-degenerate stream: the model does not just repeat a few tokens
    assert len(set(np.array(stream).reshape(-1).tolist())) > 20


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_cfg1_large_margin_variant_streams_identical(dev, kv_int8):
    """The cfg1 workload on the large-margin variant of the same 28-layer
    model (workloads.successor_model, embedding N(0, 1)): the cfg1 iteration's
    five scored rows and 64 free-running greedy steps per sequence give the
    same tokens on the device and the oracle, every step, with the logits
    inside the floor bounds.  The smallest top-2 margin seen is reported."""
    fb = floor_bounds(kv_int8)
    m = ia.SynthModel(ia.default_cfg(), seed=11, bits=2)
    try:
        wl.successor_model(m, 1.0)
        w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, m, kv_int8)
        announce(f"large-margin cfg1 kv_int8={kv_int8}: iteration")
        be, lg = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
        bo, lo = ora.forward(wl.cfg1_rows(w, dec_o, pq), logits=True)
        want = [i for i, r in enumerate(wl.cfg1_rows(w, dec_e, pe)) if r[4]]
        _check_logits(lg, lo, "large-margin cfg1", None, fb)
        assert [int(be[i]) for i in want] == [int(bo[i]) for i in want]
        seq_e, seq_o = dec_e + [pe], dec_o + [pq]
        pos = [n + 1 for n in w.contexts] + [len(w.pre_tokens)]
        tok = [int(be[i]) for i in want]
        margins, streams = [], [list(tok)]
        for step in range(64):
            announce(f"large-margin cfg1 kv_int8={kv_int8}: free-running step {step}")
            b_e, l_e = eng.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_e, pos, tok)], logits=True)
            b_o, l_o = ora.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_o, pos, tok)], logits=True)
            _check_logits(l_e, l_o, f"large-margin step {step}", None, fb)
            assert list(b_e) == list(b_o), f"step {step}: device {list(b_e)} oracle {list(b_o)}"
            srt = np.sort(l_o, axis=1)
            margins += ((srt[:, -1] - srt[:, -2]) / l_o.std(axis=1)).tolist()
            tok = [int(x) for x in b_e]
            streams.append(tok)
            pos = [p + 1 for p in pos]
        print(f"[large-margin cfg1 kv_int8={kv_int8}] 64 free-running steps identical on all 5 sequences; "
              f"top-2 margin min {min(margins):.3f} sigma, median {float(np.median(margins)):.3f}")
        out = os.environ.get("IFR_PARITY_OUT")
        if out:
            os.makedirs(out, exist_ok=True)
            with open(os.path.join(out, f"parity_cfg1_margin_kv{kv_int8}.json"), "w") as f:
                json.dump({"kv_int8": kv_int8, "steps_identical": 64, "sequences": 5,
                           "top2_margin_min": min(margins), "top2_margin_median": float(np.median(margins)),
                           "distinct_tokens": len(set(np.array(streams).reshape(-1).tolist()))}, f, indent=1)
        assert len(set(np.array(streams).reshape(-1).tolist())) > 20  # not a repeated token
    finally:
        m.close()


def _lanes(eng):
    n = C.c_int32()
    ia.check(ia.lib().ifr_debug_last_lanes(eng.dev.ctx, C.byref(n)), "lanes")
    return n.value


def test_two_lanes_match_one_lane(dev, model):
    """A forward cut into two sub-batches on the context's two streams gives
    bit-identical logits to the same forward on one stream (per-kernel
    timing runs every batch on one lane): [decode rows | prefill chunk] and
    decode rows halved."""
    cfg = model.cfg
    eng = ia.Engine(dev, model, max_seqs=24, max_seq_tokens=2048, pool_tokens=24 * 2048, max_rows=128,
                    lanes=2)
    rng = np.random.default_rng(17)
    lens = rng.integers(20, 1500, size=20).tolist()
    seqs = []
    for n in lens:
        s = eng.seq_open()
        k = rng.standard_normal((cfg.layers, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
        eng.load_kv(s, k, k)
        seqs.append(s)
    pre = eng.seq_open()
    toks = rng.integers(0, cfg.vocab, size=len(lens) + 50).tolist()
    cases = {"decode+chunk": [(s, n, toks[i], 0, 1) for i, (s, n) in enumerate(zip(seqs[:4], lens[:4]))] +
             [(pre, p, toks[20 + p], 1, int(p == 49)) for p in range(50)],
             "decode halves": [(s, n, toks[i], 0, 1) for i, (s, n) in enumerate(zip(seqs, lens))]}
    for name, rows in cases.items():
        announce(f"two lanes vs one: {name}")
        outs = []
        for timing in (True, False):
            eng.set_timing(timing)
            b, lg = eng.forward(rows, logits=True)
            outs.append((b, lg, _lanes(eng)))
            eng.set_timing(False)
            for s, n in zip(seqs, lens):
                eng.seq_truncate(s, n)
            eng.seq_truncate(pre, 0)
        (b1, l1, n1), (b2, l2, n2) = outs
        assert n1 == 1 and n2 == 2, (name, n1, n2)
        assert np.array_equal(b1, b2) and np.array_equal(l1.view(np.uint32), l2.view(np.uint32)), name


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


def test_model_load_declines_shapes_the_kernels_cannot_run(dev):
    """ifr_model_load checks every per-kernel shape limit up front: a model
    whose attention row (n_heads * head_dim = 10240) exceeds the combine
    kernel's 8192 is declined at load, not part-way through a forward."""
    cfg = ia.default_cfg(layers=1, n_heads=80, n_kv=10, inter=384, vocab=512)
    m = ia.SynthModel(cfg, seed=1, bits=2)
    try:
        announce("model load declines n_heads * head_dim > 8192")
        with pytest.raises(ia.IfrError) as e:
            ia.Engine(dev, m, max_seqs=2, max_seq_tokens=64, max_rows=16)
        assert e.value.code == ia.IFR_EDECLINE
    finally:
        m.close()
