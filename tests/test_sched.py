"""The C++ iteration scheduler (sched.cpp) without a GPU, through its backend
table (ifr_sched_create_backend).

Two backends:
  * MockLM: an exact causal "language model" in Python -- the next token is a
    hash of the sequence's token history up to the row's position, and the
    history is cut by seq_truncate.  Any correct scheduler must produce the
    same streams however it batches, splits or speculates, so the checks
    below are exact.
  * the CPU oracle forward (a8 contract) on a tiny model, for one end-to-end
    run with real numerics.

Reference behaviour restated (examples/intfer_cli/main.cpp):
  joint iteration = decode rows in live order, then <= chunk_m prefill rows of
  the prefill-queue head (sched_iteration_joint :8427-8542); split path runs
  them as two forwards (:8382-8413) and must give the same streams
  (test_cpu_parity.sh:76-92); a request finishes after max_new + 1 generated
  tokens; unfilled heads rotate round-robin (serve_rotate_unfilled
  :9187-9195); admission is gated by the live cap (serve_live_cap
  :9147-9182, admission loop :9329-9342);
  n-gram verify rows accept the longest greedy-matching draft prefix and
  truncate the KV (:11869-11915).
"""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import _abi

V = 97


class MockLM:
    """`pool` bounds the tokens held over all slots (None: unbounded), the
    way KV pages bound the engine: a forward or copy that would exceed it is
    refused with IFR_ENOMEM and changes nothing.  `copy` installs the
    seq_copy_prefix callback (prefix reuse)."""

    def __init__(self, slots=16, cap=4096, copy=True, pool=None):
        self.hist = {}
        self.free = list(range(slots))
        self.forwards = []
        self.copies = []
        self.pool = pool
        self._cb = (_abi.SEQ_OPEN(self._open), _abi.SEQ_CLOSE(self._close),
                    _abi.SEQ_TRUNC(self._trunc), _abi.FORWARD(self._fwd))
        self._copy_cb = _abi.SEQ_COPY(self._copy) if copy else _abi.SEQ_COPY()
        self._logits_cb = _abi.FORWARD_LOGITS(self._fwd_logits)
        self.table = _abi.SchedBackend(None, *self._cb, cap, self._copy_cb, self._logits_cb, V)

    def used(self):
        return sum(len(h) for h in self.hist.values())

    def _copy(self, user, dst, src, n):
        if dst not in self.hist or src not in self.hist or self.hist[dst] or n > len(self.hist[src]):
            return ia.IFR_EINVAL
        if self.pool is not None and self.used() + n > self.pool:
            return ia.IFR_ENOMEM
        self.hist[dst] = self.hist[src][:n]
        self.copies.append((dst, src, n))
        return 0

    def _open(self, user, slot):
        if not self.free:
            return ia.IFR_ENOMEM
        s = self.free.pop(0)
        self.hist[s] = []
        slot[0] = s
        return 0

    def _close(self, user, s):
        self.hist.pop(s, None)
        self.free.append(s)
        self.free.sort()
        return 0

    def _trunc(self, user, s, n):
        self.hist[s] = self.hist[s][:n]
        return 0

    @staticmethod
    def next_token(h):
        x = 1469598103
        for t in h:
            x = ((x ^ t) * 1099511) % 4294967291
        return x % V

    @staticmethod
    def logits_of(h):
        """The mock's logits after history h (returned for want = 2 rows)."""
        return (np.random.default_rng(MockLM.next_token(h) * 7919 + len(h)).standard_normal(V) * 2).astype(
            np.float32)

    def _fwd_logits(self, user, rows, M, best, logits):
        r = self._fwd(user, rows, M, best)
        if r == 0:
            k = 0
            for i, (s, p, t, kind, w) in enumerate(self.forwards[-1]):
                if w == 2:
                    lg = self.logits_of(self.hist[s][:p + 1])
                    C.memmove(C.addressof(logits.contents) + k * V * 4, lg.ctypes.data, V * 4)
                    k += 1
        return r

    def _fwd(self, user, rows, M, best):
        rs = [(rows[i].seq, rows[i].pos, rows[i].token, rows[i].kind, rows[i].want) for i in range(M)]
        if self.pool is not None and self.used() + M > self.pool:
            return ia.IFR_ENOMEM
        self.forwards.append(rs)
        for i, (s, p, t, k, w) in enumerate(rs):
            h = self.hist[s]
            if p != len(h):
                return ia.IFR_EINVAL  # rows must extend the sequence contiguously
            h.append(t)
            best[i] = self.next_token(h) if w else -1
        return 0


def run(prompts, max_new, **kw):
    lm = MockLM()
    sch = ia.Scheduler(backend=lm.table, **kw)
    ids = [sch.submit(p, max_new) for p in prompts]
    for _ in range(5000):
        n = sch.step()
        if n == 0 and all(sch.result(i)[1] for i in ids):
            break
    out = [sch.result(i)[0] for i in ids]
    sch.close()
    return out, lm


def expected_stream(prompt, max_new):
    h = list(prompt)
    out = []
    for _ in range(max_new + 1):
        t = MockLM.next_token(h)
        out.append(t)
        h.append(t)
    return out


def prompts_of(n, seed, lo=5, hi=70):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, V, size=int(rng.integers(lo, hi))).tolist() for _ in range(n)]


def test_streams_equal_greedy_history_model():
    ps = prompts_of(6, 1)
    out, lm = run(ps, 9, chunk_m=16, live_cap=8)
    assert out == [expected_stream(p, 9) for p in ps]
    assert all(len(o) == 10 for o in out)  # finish after max_new + 1 tokens


def test_split_equals_joint():
    ps = prompts_of(7, 2)
    a, la = run(ps, 11, chunk_m=24, live_cap=8, split_iter=0)
    b, lb = run(ps, 11, chunk_m=24, live_cap=8, split_iter=1)
    assert a == b
    assert any(len({r[3] for r in f}) > 1 for f in la.forwards)   # joint mixes kinds
    assert all(len({r[3] for r in f}) == 1 for f in lb.forwards)  # split never does


def test_solo_equals_loaded():
    ps = prompts_of(8, 3)
    loaded, _ = run(ps, 7, chunk_m=32, live_cap=8)
    for i in (0, 5):
        solo, _ = run([ps[i]], 7, chunk_m=32, live_cap=8)
        assert solo[0] == loaded[i]


def test_row_list_structure_and_budgets():
    ps = prompts_of(10, 4, lo=30, hi=90)
    chunk, cap = 16, 4
    _, lm = run(ps, 5, chunk_m=chunk, live_cap=cap)
    for f in lm.forwards:
        kinds = [r[3] for r in f]
        # decode rows first (live order), then the prefill rows of one request
        n_dec = sum(1 for k in kinds if k == ia.ROW_DECODE)
        assert all(k == ia.ROW_DECODE for k in kinds[:n_dec])
        pre = [r for r in f if r[3] == ia.ROW_PREFILL]
        assert len(pre) <= chunk
        assert len({r[0] for r in pre}) <= 1
        assert [r[1] for r in pre] == list(range(pre[0][1], pre[0][1] + len(pre))) if pre else True
        # the live cap gates admission only (main.cpp:9329-9342 admits while
        # live.size() < cap; requests still in prefill are not "live"), so
        # the decode row count is bounded by the requests, not by the cap
        assert n_dec <= len(ps)
        if pre:  # only the last row of a chunk can be scored (finished prompt)
            assert all(r[4] == 0 for r in pre[:-1])


def test_pack_prefill_keeps_streams_and_fills_chunks():
    """pack_prefill (no reference counterpart) fills the chunk budget from
    several queued prompts; every stream is unchanged and the iteration count
    drops, with every prefill chunk full while enough prompt rows wait."""
    ps = prompts_of(12, 21, lo=10, hi=120)
    chunk = 64
    a, la = run(ps, 6, chunk_m=chunk, live_cap=8)
    b, lb = run(ps, 6, chunk_m=chunk, live_cap=8, pack_prefill=1)
    c, lc = run(ps, 6, chunk_m=chunk, live_cap=8, pack_prefill=1, split_iter=1)
    assert a == b == c
    assert len(lb.forwards) < len(la.forwards)
    pre = [sum(1 for r in f if r[3] == ia.ROW_PREFILL) for f in lb.forwards]
    total = sum(len(p) for p in ps)
    full = total // chunk
    assert pre[:full] == [chunk] * full  # all 12 prompts are queued from the first step
    # a chunk may now carry several requests, each one contiguous
    multi = [f for f in lb.forwards if len({r[0] for r in f if r[3] == ia.ROW_PREFILL}) > 1]
    assert multi
    for f in multi:
        seqs = [r[0] for r in f if r[3] == ia.ROW_PREFILL]
        assert all(seqs[i] == seqs[i + 1] or seqs[i + 1] not in seqs[:i + 1] for i in range(len(seqs) - 1))


def test_round_robin_rotates_unfilled_heads():
    ps = [list(range(60)), list(range(1, 61)), list(range(2, 62))]
    _, lm = run(ps, 2, chunk_m=16, live_cap=8, round_robin=1)
    heads = [next(r[0] for r in f if r[3] == ia.ROW_PREFILL) for f in lm.forwards
             if any(r[3] == ia.ROW_PREFILL for r in f)]
    # the first three chunks come from three different requests
    assert len(set(heads[:3])) == 3
    _, lm2 = run(ps, 2, chunk_m=16, live_cap=8, round_robin=0)
    heads2 = [next(r[0] for r in f if r[3] == ia.ROW_PREFILL) for f in lm2.forwards
              if any(r[3] == ia.ROW_PREFILL for r in f)]
    assert heads2[:4] == [heads2[0]] * 4  # FIFO: the head fills before the next starts


def test_spec_verify_rows_keep_stream_and_accept():
    # repetitive prompts make n-gram drafts frequent; the mock's continuation
    # is deterministic, so accepted drafts must reproduce the plain stream
    base = list(range(3, 23))
    ps = [base * 3 + base[:4], base[5:] * 2, prompts_of(1, 9)[0]]
    plain, _ = run(ps, 24, chunk_m=32, live_cap=8, spec_k=0)
    spec, lm = run(ps, 24, chunk_m=32, live_cap=8, spec_k=4)
    assert spec == plain
    ver = [r for f in lm.forwards for r in f if r[3] == ia.ROW_VERIFY]
    assert ver, "no verify rows were scheduled"


def test_spec_adapt_reproduces_fixed_width_rounds():
    """SpecAdapt (main.cpp:11454-11511) picks the width maximising
    w * accept_ema / (w + 1) over 1..cap.  Without producer scores that
    ratio grows with w for any accept rate in [0.05, 0.95], so every round
    drafts up to the cap whatever the EMA has seen: a spec_adapt run issues
    exactly the forwards of the fixed-width run with spec_k = cap, and with
    spec_k = 0 the cap is 8 (main.cpp:11512-11514)."""
    base = list(range(3, 23))
    ps = [base * 3 + base[:4], base[5:] * 2, prompts_of(1, 9)[0]]
    plain, _ = run(ps, 24, chunk_m=32, live_cap=8)
    fixed3, lf = run(ps, 24, chunk_m=32, live_cap=8, spec_k=3)
    adapt3, la = run(ps, 24, chunk_m=32, live_cap=8, spec_k=3, spec_adapt=1)
    assert adapt3 == fixed3 == plain
    assert la.forwards == lf.forwards
    fixed8, l8 = run(ps, 24, chunk_m=32, live_cap=8, spec_k=8)
    adapt8, la8 = run(ps, 24, chunk_m=32, live_cap=8, spec_k=0, spec_adapt=1)
    assert adapt8 == plain
    assert la8.forwards == l8.forwards
    widths = []
    for f in la8.forwards:
        for sq in {r[0] for r in f if r[3] == ia.ROW_VERIFY}:
            widths.append(sum(1 for r in f if r[0] == sq) - 1)
    assert widths and max(widths) == 8


class DecliningLM(MockLM):
    """Declines (IFR_EDECLINE, nothing done) any forward that mixes decode
    and prefill rows, as a backend whose joint batch is too large would."""

    def _fwd(self, user, rows, M, best):
        kinds = {rows[i].kind for i in range(M)}
        if ia.ROW_PREFILL in kinds and len(kinds) > 1:
            self.declined = getattr(self, "declined", 0) + 1
            return ia.IFR_EDECLINE
        return super()._fwd(user, rows, M, best)


def test_declined_joint_forward_runs_the_split_path():
    """serve_iteration (main.cpp:9247-9256): a joint forward that declines
    has changed nothing, and the same iteration runs the split path (the
    chunk, then the decode rows), so the streams are unchanged."""
    ps = prompts_of(7, 2)
    ref, _ = run(ps, 11, chunk_m=24, live_cap=8)
    lm = DecliningLM()
    sch = ia.Scheduler(backend=lm.table, chunk_m=24, live_cap=8)
    ids = [sch.submit(p, 11) for p in ps]
    for _ in range(5000):
        if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
            break
    out = [sch.result(i)[0] for i in ids]
    sch.close()
    assert out == ref
    assert getattr(lm, "declined", 0) > 0
    assert all(len({r[3] for r in f}) == 1 for f in lm.forwards)


def expected_sampled(prompt, max_new, seed, T, k, p):
    """A sampling request's stream: the prompt's last row scores the argmax
    (main.cpp:8522-8523), then every decode token is the oracle's sample()
    over the mock's logits with the request's mt19937."""
    from oracle import pyoracle as po
    from oracle.pyoracle import ptr
    O = po.oracle()
    g = O.or_rng_create(seed)
    try:
        h = list(prompt)
        out = [MockLM.next_token(h)]
        while len(out) < max_new + 1:
            h.append(out[-1])
            out.append(O.or_sample(ptr(MockLM.logits_of(h)), V, k, p, T, g))
    finally:
        O.or_rng_free(g)
    return out


@pytest.mark.parametrize("split,spec_k", [(0, 0), (1, 0), (0, 3)])
def test_sampled_requests_follow_the_reference_sampler(split, spec_k):
    """Per-request temperature / top_k / top_p with the request's own
    mt19937 (its seed, else the scheduler's seed + id, main.cpp:9305) beside
    greedy requests, in joint, split and speculating schedulers: every stream
    is the oracle sampler's, whatever the batching; sampled requests get no
    verify rows."""
    ps = prompts_of(5, 21)
    params = [(0.8, 0, 0.0, None), (1.2, 10, 0.0, 77), (0.7, 0, 0.9, None), None, (1.0, 5, 0.8, 5)]
    lm = MockLM()
    sch = ia.Scheduler(backend=lm.table, chunk_m=16, live_cap=8, split_iter=split, spec_k=spec_k, seed=1000)
    ids = []
    for pr, pa in zip(ps, params):
        if pa is None:
            ids.append(sch.submit(pr, 9))
        else:
            T, k, pp, sd = pa
            ids.append(sch.submit(pr, 9, temperature=T, top_k=k, top_p=pp, seed=sd))
    for _ in range(2000):
        if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
            break
    for rid, pr, pa in zip(ids, ps, params):
        got = sch.result(rid)[0]
        if pa is None:
            assert got == expected_stream(pr, 9)
        else:
            T, k, pp, sd = pa
            assert got == expected_sampled(pr, 9, 1000 + rid if sd is None else sd, T, k, pp), rid
    sch.close()
    sampled_slots = set()
    for f in lm.forwards:
        for r in f:
            if r[4] == 2:
                sampled_slots.add(r[0])
                assert r[3] == ia.ROW_DECODE
    assert sampled_slots


def test_sampling_needs_a_logits_forward():
    lm = MockLM()
    lm.table.forward_logits = _abi.FORWARD_LOGITS()
    sch = ia.Scheduler(backend=lm.table, chunk_m=16, live_cap=8)
    try:
        with pytest.raises(ia.IfrError) as e:
            sch.submit([1, 2, 3], 4, temperature=0.9)
        assert e.value.code == ia.IFR_EDECLINE
        assert "forward_logits" in str(e.value)  # the library's own message, not a stale one
        sch.submit([1, 2, 3], 4)  # greedy is still accepted
    finally:
        sch.close()


def test_oracle_backend_split_equals_joint():
    """Real numerics: the CPU a8 oracle forward as the scheduler's model."""
    from oracle import pyoracle as po
    cfg = ia.default_cfg(hidden=256, layers=2, n_heads=4, n_kv=2, inter=384, vocab=512)
    model = ia.SynthModel(cfg, seed=7, bits=2)
    streams = []
    try:
        for split in (0, 1):
            ora = po.OracleEngine(model, mode=0, max_seqs=8)
            cbs = (_abi.SEQ_OPEN(lambda u, s: (s.__setitem__(0, ora.seq_open()), 0)[1]),
                   _abi.SEQ_CLOSE(lambda u, s: (ora.seq_close(s), 0)[1]),
                   _abi.SEQ_TRUNC(lambda u, s, n: (ora.seq_truncate(s, n), 0)[1]),
                   _abi.FORWARD(lambda u, rows, M, best: _ora_fwd(ora, rows, M, best)))
            table = _abi.SchedBackend(None, *cbs, 2048)
            sch = ia.Scheduler(backend=table, chunk_m=16, live_cap=4, split_iter=split)
            rng = np.random.default_rng(3)
            ids = [sch.submit(rng.integers(0, 512, size=n).tolist(), 6) for n in (9, 23, 40)]
            for _ in range(200):
                if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                    break
            streams.append([sch.result(i)[0] for i in ids])
            sch.close()
            ora.close()
    finally:
        model.close()
    assert streams[0] == streams[1]
    assert all(len(s) == 7 for s in streams[0])


def _ora_fwd(ora, rows, M, best):
    arr = (ia.Row * M)(*[rows[i] for i in range(M)])
    b = ora.forward(arr)
    for i in range(M):
        best[i] = int(b[i])
    return 0
