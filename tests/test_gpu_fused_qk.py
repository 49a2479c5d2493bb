"""The QKV projection with the q/k norm + RoPE + KV append as its epilogue
(one launch where the GEMM's launch shape holds one head per workgroup)
against the two separate passes (ifr_kv_cfg.separate_qk = 1), on the 0.8B
shape: the logits of a 300-row prefill and of the decode steps after it are
bit-identical, with fp16 and with int8 KV.  A model without q/k norm
weights (qk_norm = 0) runs the epilogue without the norm, bit-identical to
the separate pass (regression: the epilogue once read the absent weights)."""
import numpy as np
import pytest

import intfer_amd as ia
from tests.conftest import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv8,qkn", [(0, 1), (1, 1), (0, 0)])
def test_fused_qk_epilogue_bit_identical(dev, kv8, qkn):
    cfg = ia.default_cfg(layers=2, qk_norm=qkn)
    m = ia.SynthModel(cfg, seed=17, bits=2)
    try:
        rng = np.random.default_rng(31)
        prompt = rng.integers(0, cfg.vocab, size=300).tolist()
        outs = []
        for sep in (0, 1):
            announce(f"fused q/k epilogue kv_int8={kv8} qk_norm={qkn} separate={sep}: 300-row prefill + 2 decode steps")
            eng = ia.Engine(dev, m, max_seqs=4, max_seq_tokens=1024, pool_tokens=4 * 1024, kv_int8=kv8,
                            max_rows=320, separate_qk=sep)
            s = eng.seq_open()
            eng.set_timing(True)
            b, lg = eng.forward([(s, p, t, ia.ROW_PREFILL, int(p % 60 == 59)) for p, t in enumerate(prompt)],
                                logits=True)
            assert (eng.timing("qk_rope_kv")[1] > 0) == bool(sep)
            eng.set_timing(False)
            got = [lg]
            t, pos = int(b[-1]), 300
            for _ in range(2):
                b2, l2 = eng.forward([(s, pos, t, ia.ROW_DECODE, 1)], logits=True)
                got.append(l2)
                t, pos = int(b2[0]), pos + 1
            outs.append(got)
            eng.seq_close(s)
        for a, b in zip(*outs):
            assert np.array_equal(a, b)
    finally:
        m.close()
