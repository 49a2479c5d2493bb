"""The serve loop on the device engine.

  * ifr_serve over pipes streams, per request, exactly the tokens the
    scheduler produces when driven directly (generated[1:], the prefill's
    token not streamed), on a two-layer 0.8B-shaped model;
  * the intfer_serve command line under the cfg4 load harness
    (intfer_amd/serve_load.py, levels 1 / 4 / 8): every request finishes,
    the first request's stream under load equals its solo stream, and that
    stream equals the in-process one for the same prompt (same model seed).
"""
import json

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import serve_load
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MAX_NEW = 8


@pytest.fixture(scope="module")
def small():
    cfg = ia.default_cfg(layers=2)
    m = ia.SynthModel(cfg, seed=11, bits=2)
    yield cfg, m
    m.close()


def _direct(eng, prompts):
    sch = ia.Scheduler(eng, chunk_m=128, live_cap=64)
    ids = [sch.submit(p, MAX_NEW) for p in prompts]
    for _ in range(10000):
        if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
            break
    out = [sch.result(i)[0] for i in ids]
    sch.close()
    return out


def test_serve_streams_equal_direct_scheduler(dev, small):
    cfg, m = small
    eng = ia.Engine(dev, m, max_seqs=16, max_seq_tokens=4096, max_rows=256)
    prompts = serve_load.cfg4_prompts(6, seed=5, vocab=cfg.vocab, lo=16, hi=300)
    announce("serve loop vs direct scheduler, 6 requests")
    direct = _direct(eng, prompts)
    sch = ia.Scheduler(eng, chunk_m=128, live_cap=64)
    try:
        out, rc = sch.serve([json.dumps({"prompt_ids": p, "max_new": MAX_NEW}) for p in prompts],
                            vocab=cfg.vocab)
    finally:
        sch.close()
    assert rc == 0
    toks = {}
    done = {}
    for ev in out:
        assert "error" not in ev, ev
        if "token" in ev:
            toks.setdefault(ev["id"], []).append(ev["token"])
        elif ev.get("done"):
            done[ev["id"]] = ev["generated"]
    assert done == {i + 1: MAX_NEW + 1 for i in range(6)}
    for i, d in enumerate(direct):
        assert toks[i + 1] == d[1:], f"request {i + 1}"


def test_cli_serve_load_and_cross_process_parity(dev, small, tmp_path):
    cfg, m = small
    announce("intfer_serve under the cfg4 harness, levels 1 4 8")
    res = serve_load.sweep(["--synth", "11", "--layers", "2", "--max-seq-tokens", "4096",
                            "--chunk-m", "512"], levels=[1, 4, 8], max_new=MAX_NEW,
                           timeout=300, log_path=str(tmp_path / "serve.log"))
    print(json.dumps(res["levels"]))
    assert not res["fails"], (res["fails"], (tmp_path / "serve.log").read_text()[-2000:])
    # the same first prompt through the in-process engine
    eng = ia.Engine(dev, m, max_seqs=4, max_seq_tokens=4096, max_rows=640)
    first = serve_load.cfg4_prompts(8, vocab=cfg.vocab)[0]
    sch = ia.Scheduler(eng, chunk_m=512, live_cap=64)
    try:
        out, rc = sch.serve([json.dumps({"prompt_ids": first, "max_new": MAX_NEW, "id": 1})])
    finally:
        sch.close()
    mine = [ev["token"] for ev in out if "token" in ev]
    assert len(mine) == MAX_NEW and res["levels"][-1]["parity"]
    assert mine == res["solo_stream"]
    assert res["solo"]["all_done"]
