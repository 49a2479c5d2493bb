"""ifr_attention_noalloc: the attention entry point that allocates nothing
(its intermediates live in the library's fixed per-GPU device array) gives
bit-identical outputs to ifr_attention on the same rows, on two calls in a
row, the second smaller than the first (so leftovers of the first call in the
shared array would show), with fp16 and int8 KV; inputs beyond its stated
limits are refused with IFR_EINVAL."""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from tests.conftest import announce

pytestmark = pytest.mark.gpu

L = ia.lib()


def _noalloc(dev, eng, rows, q):
    arr = ia.rows_array(rows)
    M = len(arr)
    qd = dev.upload(np.ascontiguousarray(q, dtype=np.float16))
    od = dev.alloc(M * eng.cfg.n_heads * eng.cfg.head_dim * 4)
    try:
        rc = L.ifr_attention_noalloc(dev.ctx, 0, arr, M, qd.p, od.p)
        out = dev.download(od, np.float32, (M, eng.cfg.n_heads * eng.cfg.head_dim)) if rc == 0 else None
    finally:
        qd.free()
        od.free()
    return rc, out


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_noalloc_attention_matches_ifr_attention(dev, kv_int8):
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = ia.SynthModel(cfg, seed=5)
    try:
        rng = np.random.default_rng(71 + kv_int8)
        lens = rng.integers(40, 1400, size=20).tolist()
        chunk_off = 300
        eng = ia.Engine(dev, model, max_seqs=24, max_seq_tokens=2048, pool_tokens=24 * 2048,
                        kv_int8=kv_int8, max_rows=1200)
        seqs = []
        for n in lens + [chunk_off + 100]:
            s = eng.seq_open()
            k = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
            v = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
            eng.load_kv(s, k, v)
            seqs.append(s)
        big = [(seqs[i], n - 1, 0, 0, 1) for i, n in enumerate(lens)]
        big += [(seqs[-1], chunk_off + p, 0, 1, 1) for p in range(100)]
        small = [(seqs[i], lens[i] - 1, 0, 0, 1) for i in range(5)]
        small += [(seqs[-1], chunk_off + p, 0, 1, 1) for p in range(10)]
        for name, rows in (("first (120 rows)", big), ("second (15 rows)", small)):
            q = rng.standard_normal((len(rows), cfg.n_heads, cfg.head_dim), dtype=np.float32).astype(np.float16)
            announce(f"no-alloc attention kv_int8={kv_int8}: {name}")
            rc, got = _noalloc(dev, eng, rows, q)
            assert rc == ia.IFR_OK, ia.lib().ifr_last_error()
            ref = eng.attention(0, rows, q)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
        # beyond the limits: refused, with a message
        announce(f"no-alloc attention kv_int8={kv_int8}: refusal of 513 rows")
        over = [(seqs[-1], p, 0, 1, 1) for p in range(chunk_off + 100)]
        for i, n in enumerate(lens):
            over += [(seqs[i], p, 0, 1, 1) for p in range(min(n, 513 - len(over)))]
        assert len(over) == 513
        qo = np.zeros((len(over), cfg.n_heads, cfg.head_dim), np.float16)
        rc, _ = _noalloc(dev, eng, over, qo)
        assert rc == ia.IFR_EINVAL and b"no-allocation limit" in ia.lib().ifr_last_error()
        del eng
    finally:
        model.close()


def test_noalloc_refuses_more_units_than_its_scratch(dev):
    """A batch within the row limit whose attention units exceed the 4096 the
    scratch holds: 512 rows of one sequence at positions 1536..2047 are 64
    q-blocks x 8 kv heads x 13..16 KV splits of 128 tokens (7424 units).
    Refused with IFR_EINVAL and a message, before any kernel runs."""
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = ia.SynthModel(cfg, seed=5)
    try:
        eng = ia.Engine(dev, model, max_seqs=2, max_seq_tokens=2048, pool_tokens=2 * 2048, max_rows=512,
                        attn_split=128)
        rng = np.random.default_rng(9)
        s = eng.seq_open()
        eng.load_kv(s, rng.standard_normal((1, 2048, cfg.n_kv, cfg.head_dim), dtype=np.float32),
                    rng.standard_normal((1, 2048, cfg.n_kv, cfg.head_dim), dtype=np.float32))
        rows = [(s, 1536 + p, 0, 1, 1) for p in range(512)]
        announce("no-alloc attention: refusal of 7424 units in 512 rows")
        rc, _ = _noalloc(dev, eng, rows, np.zeros((512, cfg.n_heads, cfg.head_dim), np.float16))
        assert rc == ia.IFR_EINVAL and b"attention units" in ia.lib().ifr_last_error()
        del eng
    finally:
        model.close()


def test_noalloc_calls_from_two_contexts_wait_for_each_other():
    """Two contexts on the one GPU, each with its own engine, call
    ifr_attention_noalloc from two threads at once, 12 times each with
    different batches: every result equals its own context's ifr_attention,
    bit for bit (the calls share the GPU's scratch array and are serialized
    by the library's per-device lock)."""
    import threading
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = ia.SynthModel(cfg, seed=9)
    devs = [ia.Device(0), ia.Device(0)]
    try:
        jobs = []
        for di, d in enumerate(devs):
            rng = np.random.default_rng(500 + di)
            eng = ia.Engine(d, model, max_seqs=8, max_seq_tokens=2048, pool_tokens=8 * 2048, max_rows=512)
            seqs = []
            for n in (300 + 200 * di, 900, 1500 - 100 * di, 700):
                s = eng.seq_open()
                k = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
                v = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
                eng.load_kv(s, k, v)
                seqs.append((s, n))
            cases = []
            for it in range(12):
                rows = [(s, n - 1 - it, 0, 0, 1) for s, n in seqs[:3]]
                rows += [(seqs[3][0], 500 + p, 0, 1, 1) for p in range(40 + 10 * it)]
                q = rng.standard_normal((len(rows), cfg.n_heads, cfg.head_dim), dtype=np.float32).astype(np.float16)
                cases.append((rows, q, eng.attention(0, rows, q)))
            jobs.append((d, eng, cases))
        errors = []

        def run(d, eng, cases):
            for i, (rows, q, ref) in enumerate(cases):
                rc, got = _noalloc(d, eng, rows, q)
                if rc != ia.IFR_OK or not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
                    errors.append((d, i, rc))

        announce("no-alloc attention: two contexts, two threads, 12 calls each")
        th = [threading.Thread(target=run, args=j) for j in jobs]
        for t in th:
            t.start()
        for t in th:
            t.join()
        assert not errors, errors
        del jobs
    finally:
        for d in devs:
            d.close()
        model.close()
