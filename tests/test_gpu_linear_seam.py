"""The per-linear seam (LinearBackend, examples/intfer_cli/main.cpp:455-566)
on the device: ifr_linear_batch / ifr_linear_wave_batch / ifr_mlp_fused over
the loaded model's linears, host fp32 rows in and out.

  * every linear of two layers (Q, K, V out of the fused QKV projection,
    gate and up out of the interleaved pair, O, down), at M = 1, 37 and
    300 (two chunks of the engine's 256-row workspace), equals the oracle's
    restatement of the contract bit for bit: per-token int8 quantization of
    each input row, int32 T, the fp32 group fold, fp16 output read back as
    fp32 (the reference GPU backend's half_to_float);
  * the wave of independent linears equals the linears one by one;
  * the fused MLP equals the oracle's gate/up -> fp16 silu(g) * u ->
    per-token quantization -> down on every row where the device expf of
    the SwiGLU gives the fp16 value the host's does (it may differ by one
    fp16 ulp, moving an int8 code of the down projection's input);
  * the reference tensor names map to (layer, linear), the rotation site of
    each linear is the reference's (right for q/k/v/gate/up, left for
    o/down), and names outside the model are refused.
"""
import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from tests.conftest import announce

pytestmark = pytest.mark.gpu

NAMES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
         "mlp.up_proj", "mlp.down_proj")


class _Lin:
    def __init__(self, s):
        self.struct, self.N, self.K = s, s.N, s.K


def _ref_linear(lin, X):
    q, sc, _ = po.act_quant(X)
    return po.qgemm(q, sc[:, 0], _Lin(lin)).view(np.float16).astype(np.float32)


@pytest.fixture(scope="module")
def setup(dev):
    cfg = ia.default_cfg(layers=2)
    m = ia.SynthModel(cfg, seed=21, bits=2)
    eng = ia.Engine(dev, m, max_seqs=2, max_seq_tokens=256, max_rows=256)
    yield cfg, m, eng
    del eng
    m.close()


def test_every_linear_matches_the_contract(setup):
    cfg, m, eng = setup
    rng = np.random.default_rng(3)
    for l in (0, 1):
        lw = m.layer(l)
        for which, nm in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
            lin = getattr(lw, nm)
            assert eng.linear_shape(l, which) == (lin.N, lin.K)
            for M in (1, 37, 300):
                X = rng.standard_normal((M, lin.K), dtype=np.float32)
                announce(f"linear seam layer {l} {nm} M={M}")
                Y = eng.linear_batch(l, which, X)
                assert np.array_equal(Y.view(np.uint32), _ref_linear(lin, X).view(np.uint32)), (l, nm, M)


def test_wave_equals_single_linears(setup):
    cfg, m, eng = setup
    rng = np.random.default_rng(4)
    M = 45
    items = [(1, w, rng.standard_normal((M, eng.linear_shape(1, w)[1]), dtype=np.float32)) for w in range(7)]
    announce("linear seam wave of 7 linears")
    ys = eng.linear_wave_batch(items, M)
    for (l, w, X), Y in zip(items, ys):
        assert np.array_equal(Y.view(np.uint32), eng.linear_batch(l, w, X).view(np.uint32)), w


def test_mlp_fused_matches_the_contract(setup):
    cfg, m, eng = setup
    rng = np.random.default_rng(5)
    M, H, F = 300, cfg.hidden, cfg.inter
    rin = rng.standard_normal((M, H), dtype=np.float32)
    announce(f"linear seam fused MLP M={M}")
    md = eng.mlp_fused(0, rin)
    lw = m.layer(0)
    q, sc, _ = po.act_quant(rin)
    g = po.qgemm(q, sc[:, 0], _Lin(lw.gate))
    u = po.qgemm(q, sc[:, 0], _Lin(lw.up))
    mg = np.empty_like(g)
    po.oracle().or_swiglu(po.ptr(g), po.ptr(u), po.ptr(mg), g.size)
    ref = _ref_linear(lw.down, mg.view(np.float16).astype(np.float32))
    exact = sum(np.array_equal(md[r].view(np.uint32), ref[r].view(np.uint32)) for r in range(M))
    dmax = float(np.abs(md - ref).max())
    print(f"[mlp fused] rows bit-identical {exact}/{M}, max |d| {dmax:.3g} (rms of md {float(np.sqrt((ref ** 2).mean())):.3g})")
    assert exact >= 0.9 * M and dmax <= 0.05 * float(np.abs(ref).max())


def test_names_shapes_and_rotation_sites(setup):
    cfg, m, eng = setup
    for l in (0, 1):
        for w, nm in enumerate(NAMES):
            assert eng.linear_lookup(f"model.language_model.layers.{l}.{nm}.weight") == (l, w)
    assert [eng.linear_rot(w) for w in range(7)] == [1, 1, 1, 2, 1, 1, 2]
    for bad in ("model.language_model.layers.2.self_attn.q_proj.weight",  # beyond the model
                "model.language_model.layers.0.self_attn.q_norm.weight",  # not a linear
                "lm_head.weight", "model.language_model.layers.x.mlp.up_proj.weight"):
        with pytest.raises(ia.IfrError) as e:
            eng.linear_lookup(bad)
        assert e.value.code == ia.IFR_EINVAL
