"""cfg5 shape family on the device: the 27B-class layer (hidden 5120, 40 q /
8 kv heads so a GQA group of 5, FFN 17408, a seeded per-tensor 70 % INT2 /
30 % INT4 split, INT8 KV) against the CPU oracle on a reduced batch of the
cfg5 kinds: decode rows, n-gram verify groups (a token plus 4 drafts) and a
causal prefill chunk.  One layer and 152 rows keep the oracle's CPU time in
seconds; the full 64-layer, M ~ 2160 iteration is measured by
`bench.py --cfg5`.

Bounds: the model-level bounds of test_gpu_forward (rms <= 0.25 sigma,
corr >= 0.97, max <= 1.5 sigma per logit row) and the same greedy tokens on
every scored row but at most one (a row whose top-2 margin is below the
error difference may flip).
"""
import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from oracle import pyoracle as po
from tests.conftest import announce
from tests.test_gpu_forward import _check_logits

pytestmark = pytest.mark.gpu


def test_cfg5_layer_mixed_rows(dev):
    cfg = ia.default_cfg(hidden=5120, layers=1, n_heads=40, n_kv=8, inter=17408)
    m = ia.SynthModel(cfg, seed=27, bits=0)
    try:
        eng = ia.Engine(dev, m, max_seqs=16, max_seq_tokens=4608, pool_tokens=16 * 4608, kv_int8=1,
                        max_rows=256)
        ora = po.OracleEngine(m, kv_int8=1, mode=0, max_seqs=16)
        rng = np.random.default_rng(55)
        ctx = rng.integers(512, 4097, size=8).tolist()
        se, so = [], []
        for n in ctx:
            k, v = wl.seeded_kv(rng, 1, n, cfg.n_kv, cfg.head_dim)
            s = eng.seq_open()
            eng.load_kv(s, k, v)
            se.append(s)
            kr = k.astype(np.float16).astype(np.float32).reshape(-1, cfg.head_dim)
            vr = v.astype(np.float16).astype(np.float32).reshape(-1, cfg.head_dim)
            for arr in (kr, vr):
                for i in range(arr.shape[0]):
                    seg = np.ascontiguousarray(arr[i])
                    po.oracle().or_kv_int8_round(po.ptr(seg), cfg.head_dim)
                    arr[i] = seg
            t = ora.seq_open()
            ora.set_kv(t, kr.reshape(1, n, -1), vr.reshape(1, n, -1))
            so.append(t)
        pe, po_ = eng.seq_open(), ora.seq_open()
        toks = rng.integers(0, cfg.vocab, size=8 + 16 + 128).tolist()

        def rows(seqs, pre):
            r, i = [], 0
            for j in range(4):  # decode rows
                r.append((seqs[j], ctx[j], toks[i], ia.ROW_DECODE, 1))
                i += 1
            for j in range(4, 8):  # verify groups: token + 4 drafts
                for d in range(5):
                    r.append((seqs[j], ctx[j] + d, toks[i], ia.ROW_VERIFY, 1))
                    i += 1
            for p in range(128):  # prefill chunk of a new sequence
                r.append((pre, p, toks[i], ia.ROW_PREFILL, int(p == 127)))
                i += 1
            return r

        announce("cfg5 layer: 4 decode + 4x5 verify + 128 prefill rows, INT8 KV")
        be, lg = eng.forward(rows(se, pe), logits=True)
        bo, lo = ora.forward(rows(so, po_), logits=True)
        want = [i for i, r in enumerate(rows(se, pe)) if r[4]]
        assert len(want) == 25 and lg.shape == lo.shape == (25, cfg.vocab)
        _check_logits(lg, lo, "cfg5")
        diff = sum(1 for i in want if be[i] != bo[i])
        print(f"[cfg5] token disagreements {diff}/25, max |dlogit| {float(np.abs(lg - lo).max()):.3g}")
        assert diff <= 1
    finally:
        m.close()
