"""Prefix cache of the scheduler (ifr_sched_cfg.prefix_cache) without a GPU.

Restated from the reference's PrefixCache (examples/intfer_cli/main.cpp:
9469-9720) and its admission / completion sites (:9871-9886, :9937-9953):
  * a request that finished with its whole prompt in keeps its KV as an
    entry: stream = prompt + generated, valid for stream length - 1 positions
    (the last generated id was never forwarded);
  * at admission the longest common prefix of the new prompt with any entry
    (capped at the entry's state length and below the whole new prompt) is
    copied, and only the rest of the prompt prefills; the hit entry becomes
    the most recently used;
  * at most N entries, least recently used evicted first.
On this engine a cached entry is an open KV slot, so entries also give way
when slots or KV pages run out.  The model is the exact causal mock of
test_sched (next token = hash of the history), so every stream is known in
closed form and must be identical with and without the cache.
"""
import pytest

import intfer_amd as ia
from intfer_amd import _abi
from tests.test_sched import MockLM, expected_stream, prompts_of


def drive(sch, prompt, max_new):
    rid = sch.submit(prompt, max_new)
    for _ in range(5000):
        if sch.step() == 0 and sch.result(rid)[1]:
            break
    out, done = sch.result(rid)
    assert done
    return out


def prefill_rows(forwards, seq):
    return [r for f in forwards for r in f if r[0] == seq and r[3] == ia.ROW_PREFILL]


def test_chat_turns_resume_from_the_cached_stream():
    p1 = prompts_of(1, 21, lo=40, hi=41)[0]
    lm = MockLM(slots=8)
    sch = ia.Scheduler(backend=lm.table, chunk_m=16, live_cap=8, prefix_cache=4)
    try:
        g1 = drive(sch, p1, 6)
        assert g1 == expected_stream(p1, 6)
        # the second turn: the whole first exchange plus new user tokens
        p2 = p1 + g1 + [7, 8, 9]
        n0 = len(lm.forwards)
        g2 = drive(sch, p2, 5)
    finally:
        sch.close()
    assert g2 == expected_stream(p2, 5)
    # one copy of the 46 positions the first stream holds (47 ids, the last
    # never forwarded); only the remaining 3 + 1 prompt rows prefill
    assert len(lm.copies) == 1 and lm.copies[0][2] == len(p1) + len(g1) - 1
    rows = [r for f in lm.forwards[n0:] for r in f if r[3] == ia.ROW_PREFILL]
    assert [r[1] for r in rows] == list(range(len(p1) + len(g1) - 1, len(p2)))
    assert lm.hist == {}  # close() releases the cached slots too


def test_identical_prompt_is_capped_below_the_whole_prompt():
    p = prompts_of(1, 22, lo=30, hi=31)[0]
    lm = MockLM(slots=8)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8, prefix_cache=2)
    try:
        a = drive(sch, p, 4)
        n0 = len(lm.forwards)
        b = drive(sch, p, 4)
    finally:
        sch.close()
    assert a == b == expected_stream(p, 4)
    assert lm.copies[-1][2] == len(p) - 1
    rows = [r for f in lm.forwards[n0:] for r in f if r[3] == ia.ROW_PREFILL]
    assert [(r[1], r[4]) for r in rows] == [(len(p) - 1, 1)]


def test_streams_identical_with_and_without_cache_under_load():
    base = prompts_of(4, 23, lo=20, hi=60)
    # a mix of unrelated prompts and prompts sharing long prefixes
    ps = base + [base[0] + [1, 2, 3], base[1][:15] + [4] * 9, base[2] + base[3], base[0][:5]]
    outs = []
    for n in (0, 3):
        lm = MockLM(slots=16)
        sch = ia.Scheduler(backend=lm.table, chunk_m=16, live_cap=4, prefix_cache=n)
        try:
            first = [drive(sch, p, 7) for p in ps[:4]]   # one at a time
            ids = [sch.submit(p, 7) for p in ps[4:]]     # then together
            for _ in range(5000):
                if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                    break
            outs.append(first + [sch.result(i)[0] for i in ids])
        finally:
            sch.close()
        if n:
            assert lm.copies, "no prefix was reused"
    assert outs[0] == outs[1] == [expected_stream(p, 7) for p in ps]


def test_lru_eviction_and_promotion():
    a, b, c = prompts_of(3, 24, lo=20, hi=30)
    lm = MockLM(slots=8)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8, prefix_cache=2)
    try:
        drive(sch, a, 2)
        drive(sch, b, 2)
        assert len(lm.hist) == 2          # both kept
        drive(sch, a + [5], 2)            # hit on a: a becomes most recent
        assert lm.copies[-1][2] == len(a)  # capped below the whole prompt
        assert len(lm.hist) == 2          # a+[5] entered, b (least recent) left
        n = len(lm.copies)
        drive(sch, b + [6], 2)            # b was evicted: no hit
        assert len(lm.copies) == n
        drive(sch, c, 2)                  # entries now: c, b+[6]
        drive(sch, a + [5, 9], 2)         # a's prefix is gone: no copy
        assert len(lm.copies) == n
    finally:
        sch.close()
    assert lm.hist == {}


def test_entries_give_way_to_slots_and_pages():
    ps = prompts_of(3, 25, lo=20, hi=25)
    # two slots: the cached entry must close so the next request can open
    lm = MockLM(slots=2)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8, prefix_cache=4)
    try:
        outs = [drive(sch, p, 3) for p in ps]
    finally:
        sch.close()
    assert outs == [expected_stream(p, 3) for p in ps]
    # a token pool that holds one finished stream plus one running request
    lm = MockLM(slots=8, pool=60)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8, prefix_cache=4)
    try:
        outs = [drive(sch, p, 3) for p in ps]
    finally:
        sch.close()
    assert outs == [expected_stream(p, 3) for p in ps]


def test_backend_without_copy_runs_uncached():
    ps = prompts_of(2, 26)
    lm = MockLM(slots=4, copy=False)
    sch = ia.Scheduler(backend=lm.table, chunk_m=32, live_cap=8, prefix_cache=4)
    try:
        outs = [drive(sch, p, 3) for p in [ps[0], ps[0] + [1]]]
        assert len(lm.hist) == 0  # nothing kept open
    finally:
        sch.close()
    assert outs[1] == expected_stream(ps[0] + [1], 3)


@pytest.mark.parametrize("n", [-1, 17])
def test_prefix_cache_size_is_validated(n):
    lm = MockLM()
    with pytest.raises(_abi.IfrError):
        ia.Scheduler(backend=lm.table, prefix_cache=n)
