"""The attention output gate on the device (ifr_model_cfg.attn_gate: q_proj
rows [q, gate] per head, attn *= sigmoid(gate) before the O projection,
main.cpp:7625-7640, :7697-7698), against the CPU oracle's restatement.

  * zero gate rows (scale 0: gate = 0, sigmoid = 1/2 exactly) give the
    ungated model of the same seed with its O projection's post factor 1/2,
    bit for bit, through the whole 2-layer forward and greedy steps: the
    per-token quantization of x / 2 has the codes of x and half the scale;
  * the fused QKV epilogue and the separate q/k pass give the same bits;
  * with attn_gate_off (attn_output_gate = false) the packed model equals
    the ungated one of the same seed, bit for bit;
  * a gated one-layer model matches the oracle's tokens and logits within
    the one-layer bound (the gate's device expf may move an int8 code of the
    O-projection input by one), and the full 28-layer cfg1 iteration stays
    within the model-level bounds of test_gpu_forward."""
import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from tests.conftest import announce
from tests.test_gpu_forward import _check_logits, _setup

pytestmark = pytest.mark.gpu


def _zero_gate_pair(layers):
    cfg = ia.default_cfg(layers=layers, attn_gate=1)
    gated = ia.SynthModel(cfg, seed=11, bits=2)
    plain = ia.SynthModel(ia.default_cfg(layers=layers), seed=11, bits=2)
    for l in range(layers):
        q = gated.layer(l).q
        sc = np.ctypeslib.as_array(q.scale, shape=(q.N, q.K // 128))
        for h in range(cfg.n_heads):
            sc[(2 * h + 1) * cfg.head_dim:(2 * h + 2) * cfg.head_dim] = 0
        plain.ptr.contents.layers[l].o.post = 0.5
    return gated, plain


def _run(dev, model, prompt, steps, separate_qk=0, kv_int8=0):
    eng = ia.Engine(dev, model, max_seqs=4, max_seq_tokens=1024, max_rows=256, separate_qk=separate_qk,
                    kv_int8=kv_int8)
    try:
        s = eng.seq_open()
        n = len(prompt)
        b, lg = eng.forward([(s, p, t, ia.ROW_PREFILL, int(p % 64 == 63 or p == n - 1))
                             for p, t in enumerate(prompt)], logits=True)
        out, tok = [lg], int(b[-1])
        for i in range(steps):
            b, lg = eng.forward([(s, n + i, tok, ia.ROW_DECODE, 1)], logits=True)
            out.append(lg)
            tok = int(b[0])
        return out
    finally:
        del eng


def test_zero_gate_equals_halved_o_projection(dev):
    gated, plain = _zero_gate_pair(2)
    try:
        prompt = np.random.default_rng(31).integers(0, 151936, size=200).tolist()
        announce("zero-gate model vs halved O projection, 200-row prefill + 6 steps")
        a = _run(dev, gated, prompt, 6)
        b = _run(dev, plain, prompt, 6)
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    finally:
        gated.close()
        plain.close()


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_gate_off_equals_the_ungated_model(dev, kv_int8):
    """attn_gate_off (attn_output_gate = false, main.cpp:250, :7697) on a
    packed q_proj: the q rows come out of the [q, gate] layout and the gate
    is not applied, so the device forward equals the ungated model of the
    same seed (whose q rows are the same), bit for bit."""
    cfg_off = ia.default_cfg(layers=2, attn_gate=1, attn_gate_off=1)
    off = ia.SynthModel(cfg_off, seed=13, bits=2)
    plain = ia.SynthModel(ia.default_cfg(layers=2), seed=13, bits=2)
    try:
        prompt = np.random.default_rng(33).integers(0, 151936, size=200).tolist()
        announce(f"gate off vs ungated, kv_int8={kv_int8}")
        a = _run(dev, off, prompt, 4, kv_int8=kv_int8)
        b = _run(dev, plain, prompt, 4, kv_int8=kv_int8)
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    finally:
        off.close()
        plain.close()


def test_gated_fused_epilogue_equals_separate_pass(dev):
    m = ia.SynthModel(ia.default_cfg(layers=2, attn_gate=1), seed=12, bits=2)
    try:
        prompt = np.random.default_rng(32).integers(0, 151936, size=250).tolist()
        announce("gated model: fused QKV epilogue vs separate q/k pass")
        a = _run(dev, m, prompt, 3, separate_qk=0)
        b = _run(dev, m, prompt, 3, separate_qk=1)
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    finally:
        m.close()


@pytest.mark.parametrize("layers", [1, 28])
def test_gated_cfg1_iteration_against_oracle(dev, layers):
    m = ia.SynthModel(ia.default_cfg(layers=layers, attn_gate=1), seed=11, bits=2)
    try:
        w, eng, ora, dec_e, dec_o, pe, pq = _setup(dev, m, 0)
        announce(f"gated cfg1 iteration, {layers} layers")
        be, lg = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
        bo, lo = ora.forward(wl.cfg1_rows(w, dec_o, pq), logits=True)
        if layers == 1:
            assert np.array_equal(be, bo)
            dmax = float(np.abs(lg - lo).max())
            print(f"[gated one layer] max |dlogit| {dmax:.3g} ({dmax / float(lo.std()):.3g} sigma)")
            assert dmax <= 2e-2 * float(lo.std())
        else:
            _check_logits(lg, lo, "gated cfg1")
    finally:
        m.close()
