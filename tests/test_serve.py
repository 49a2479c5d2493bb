"""The --serve JSON-lines loop (ifr_serve, serve.cpp) without a GPU.

The loop runs over pipes on a scheduler whose model is the exact causal mock
of tests/test_sched.py (next token = hash of the sequence's history), so the
stream each request must produce is known in closed form.  Restated from
run_serve (examples/intfer_cli/main.cpp:9260-9377) and parse_serve_line
(:8595-8676):
  * one request per line; max_new defaults to 64 and is clamped to [1, 4096];
    a missing id takes the next free one (after any explicit id);
  * {"id","token"} per token of a decode row -- the token that completes the
    prefill is not streamed -- and {"id","done":true,"generated":n} with
    n = max_new + 1 once the request finishes;
  * malformed lines get {"error":...} and do not stop the loop;
  * an empty prompt falls back to the reference's canned prompt ids.
Token ids replace the reference's prompt text (no tokenizer in this build).
"""
import json

import numpy as np
import pytest

import intfer_amd as ia
from tests.test_sched import MockLM, V, expected_stream, prompts_of


def serve(lines, vocab=0, default_max_new=64, **kw):
    lm = MockLM(slots=32)
    sch = ia.Scheduler(backend=lm.table, **kw)
    try:
        out, rc = sch.serve(lines, vocab=vocab, default_max_new=default_max_new)
        info = sch.info()
    finally:
        sch.close()
    return out, rc, lm, info


def line(prompt, max_new=None, rid=None, **extra):
    d = {"prompt_ids": [int(t) for t in prompt]}
    if max_new is not None:
        d["max_new"] = max_new
    if rid is not None:
        d["id"] = rid
    d.update(extra)
    return json.dumps(d)


def streams_of(out):
    toks, done = {}, {}
    for ev in out:
        if "token" in ev:
            assert ev["id"] not in done, "token after done"
            toks.setdefault(ev["id"], []).append(ev["token"])
        elif ev.get("done"):
            done[ev["id"]] = ev["generated"]
    return toks, done


def test_streams_and_done_lines():
    ps = prompts_of(6, 11)
    out, rc, _, info = serve([line(p, 7) for p in ps], chunk_m=16, live_cap=8)
    assert rc == 0 and info[:3] == (0, 0, 0)
    toks, done = streams_of(out)
    assert sorted(done) == [1, 2, 3, 4, 5, 6]
    for i, p in enumerate(ps, start=1):
        exp = expected_stream(p, 7)
        assert toks[i] == exp[1:]  # the prefill's token is not streamed
        assert done[i] == 8        # max_new + 1 generated


def test_solo_equals_loaded_and_joint_equals_split():
    ps = prompts_of(12, 12, lo=20, hi=90)
    loaded, *_ = serve([line(p, 9) for p in ps], chunk_m=32, live_cap=8)
    split, *_ = serve([line(p, 9) for p in ps], chunk_m=32, live_cap=8, split_iter=1)
    assert streams_of(loaded) == streams_of(split)
    for i in (0, 7):
        solo, *_ = serve([line(ps[i], 9)], chunk_m=32, live_cap=8)
        assert streams_of(solo)[0][1] == streams_of(loaded)[0][i + 1]


def test_ids_defaults_and_clamps():
    p = prompts_of(1, 13)[0]
    lines = [line(p), line(p, 3, rid=40), line(p, 0), line(p, -5, rid=7), line(p, 2.9)]
    out, rc, _, _ = serve(lines, default_max_new=5, chunk_m=64, live_cap=8)
    toks, done = streams_of(out)
    # ids: 1 (auto), 40, 41 (auto after 40), 7, 42
    assert rc == 0 and sorted(done) == [1, 7, 40, 41, 42]
    assert done[1] == 6            # default max_new 5
    assert done[40] == 4
    assert done[41] == 2           # max_new 0 clamps to 1
    assert done[7] == 2            # negative clamps to 1
    assert done[42] == 3           # a real truncates, like atoi
    assert toks[40] == expected_stream(p, 3)[1:]


def test_refusals_keep_serving():
    p = prompts_of(1, 14)[0]
    lines = ["not json", '{"prompt":"hello"}', '{"max_new":3}',
             line([5, V + 1000], 2, rid=9), '{"prompt_ids":[1,"x"]}', line(p, 2, rid=3),
             line(list(range(10)) * 500, 64, rid=11)]
    out, rc, _, _ = serve(lines, vocab=V + 10, chunk_m=64, live_cap=8)
    assert rc == 0
    errs = [e for e in out if "error" in e]
    msgs = [e["error"] for e in errs]
    assert msgs.count("malformed request line") == 3
    assert any("tokenizer" in m for m in msgs)
    assert any("out of range" in m and e.get("id") == 9 for m, e in zip(msgs, errs))
    assert any("KV capacity" in m and e.get("id") == 11 for m, e in zip(msgs, errs))
    toks, done = streams_of(out)
    assert done == {3: 3} and toks[3] == expected_stream(p, 2)[1:]


def test_sampling_keys_are_served():
    """temperature / top_k / top_p / seed per line (parse_serve_line,
    main.cpp:8646-8668) over the serve defaults; a line without a seed draws
    from mt19937(serve seed + its id) (main.cpp:9305); top_k < 0 reads as 0
    and top_p is clamped to [0, 1]."""
    from tests.test_sched import expected_sampled
    ps = prompts_of(4, 31)
    lines = [line(ps[0], 6, temperature=0.8, seed=42), line(ps[1], 6, rid=20, temperature=1.1, top_k=7),
             line(ps[2], 6, top_p=0.9, top_k=-3), line(ps[3], 6)]
    lm = MockLM(slots=32)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8)
    try:
        out, rc = sch.serve(lines, default_max_new=64, temperature=0.5, seed=900)
    finally:
        sch.close()
    toks, done = streams_of(out)
    assert rc == 0 and done == {1: 7, 20: 7, 21: 7, 22: 7}
    assert toks[1] == expected_sampled(ps[0], 6, 42, 0.8, 0, 0.0)[1:]
    assert toks[20] == expected_sampled(ps[1], 6, 920, 1.1, 7, 0.0)[1:]
    assert toks[21] == expected_sampled(ps[2], 6, 921, 0.5, 0, 0.9)[1:]
    assert toks[22] == expected_sampled(ps[3], 6, 922, 0.5, 0, 0.0)[1:]


def test_empty_prompt_uses_reference_fallback():
    out, rc, lm, _ = serve(['{"prompt_ids":[],"max_new":2}'], chunk_m=64, live_cap=8)
    toks, done = streams_of(out)
    assert toks[1] == expected_stream([760, 6511, 314, 9338, 369], 2)[1:]
    assert [r[2] for r in lm.forwards[0]] == [760, 6511, 314, 9338, 369]


def test_crlf_blank_lines_and_unterminated_last_line():
    p = prompts_of(2, 15)
    lm = MockLM(slots=8)
    sch = ia.Scheduler(backend=lm.table, chunk_m=64, live_cap=8)
    try:
        raw = "\r\n".join([line(p[0], 2), "", "   ", line(p[1], 2)])
        out, rc = sch.serve([raw])
    finally:
        sch.close()
    toks, done = streams_of(out)
    assert rc == 0 and done == {1: 3, 2: 3}


def test_live_cap_counts_decoding_requests_only():
    """run_serve admits pending lines while live.size() < cap (main.cpp:
    9329-9342), and requests still filling their prompt are not live: lines
    that arrive together while nothing decodes are all admitted at once, so
    the decode width can exceed the cap."""
    ps = prompts_of(9, 16, lo=5, hi=12)
    out, rc, lm, _ = serve([line(p, 12) for p in ps], chunk_m=64, live_cap=2)
    toks, done = streams_of(out)
    assert rc == 0 and len(done) == 9
    assert all(toks[i] == expected_stream(p, 12)[1:] for i, p in enumerate(ps, start=1))
    assert max(sum(1 for r in f if r[3] == ia.ROW_DECODE) for f in lm.forwards) == 9


def test_spec_rows_stream_every_accepted_token():
    base = list(range(3, 23))
    ps = [base * 3 + base[:4], base[5:] * 2]
    plain, *_ = serve([line(p, 20) for p in ps], chunk_m=64, live_cap=8)
    spec, _, lm, _ = serve([line(p, 20) for p in ps], chunk_m=64, live_cap=8, spec_k=4)
    assert streams_of(spec) == streams_of(plain)
    assert any(r[3] == ia.ROW_VERIFY for f in lm.forwards for r in f)
