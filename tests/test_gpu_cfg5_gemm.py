"""The cfg5 (27B-class) projections at their real shapes and the real
iteration size M = 2160, through the engine's default launch shape (the
64 x 64 and 32 x 256 blocks, the XCD-grouped order and the deep K loops that
only these sizes select), against the CPU oracle on a sample and against a
second launch shape in full:

  * 24 sampled rows x the first and the last 128 output columns equal the
    oracle's GEMM contract bit for bit (the SwiGLU pair within the device
    expf's fp16 ulp, as in test_gpu_kernels);
  * the whole M x N output equals the output of another applicable launch
    shape bit for bit (every shape computes the same integer T and folds it
    in the same group order).
The oracle on all 2160 x N outputs would take minutes of CPU time; the
sampled rows and the edge columns cover every row block's and the last
column block's launch arithmetic."""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr
from tests.conftest import announce

pytestmark = pytest.mark.gpu
L = ia.lib()
M = 2160


def _rows_of(lin, lo, hi):
    """Output columns [lo, hi) of a host linear as a linear of its own."""
    rb, ng = lin.K * lin.bits // 8, lin.K // 128
    return ia.HostLinear(hi - lo, lin.K, lin.bits, lin.codes[lo * rb:hi * rb].copy(),
                         lin.scale.reshape(lin.N, ng)[lo:hi].copy().reshape(-1),
                         lin.zero.reshape(lin.N, ng)[lo:hi].copy().reshape(-1),
                         lin.values[lo:hi].copy(), lin.post)


@pytest.mark.parametrize("name,K,N,pair,other", [("qkv", 5120, 7168, False, 5), ("o", 5120, 5120, False, 5),
                                                 ("gate_up", 5120, 17408, True, 5), ("down", 17408, 5120, False, 4)])
@pytest.mark.parametrize("bits", [2, 4])
def test_cfg5_projection_full_shape(dev, name, K, N, pair, other, bits):
    rng = np.random.default_rng({"qkv": 1, "o": 2, "gate_up": 3, "down": 4}[name] * 10 + bits)
    lins = [ia.make_linear(N, K, bits, rng) for _ in range(2 if pair else 1)]
    x = rng.standard_normal((M, K), dtype=np.float32)
    q, s, g = po.act_quant(x)
    dl = C.c_void_p()
    if pair:
        ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(lins[0].struct), C.byref(lins[1].struct),
                                          C.byref(dl)), "pair")
    else:
        ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lins[0].struct), C.byref(dl)), "upload")
    qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(s[:, 0].copy()), dev.upload(g)
    od = dev.alloc(M * N * 2)
    try:
        announce(f"cfg5 {name} bits={bits} M={M} default launch shape")
        if pair:
            ia.check(L.ifr_quant_gemm_swiglu(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p), "swiglu")
        else:
            ia.check(L.ifr_quant_gemm(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, None), "gemm")
        out = dev.download(od, np.uint16, (M, N))
        announce(f"cfg5 {name} bits={bits} M={M} launch shape {other}")
        ia.check(L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, other), "variant")
        out2 = dev.download(od, np.uint16, (M, N))
        assert np.array_equal(out, out2)
        rows = np.sort(rng.choice(M, size=24, replace=False))
        for lo, hi in ((0, 128), (N - 128, N)):
            subs = [_rows_of(l, lo, hi) for l in lins]
            ref = [po.qgemm(q[rows], s[rows, 0], sl) for sl in subs]
            got = out[rows, lo:hi]
            if not pair:
                assert np.array_equal(got, ref[0]), (lo, hi)
                continue
            sw = np.empty_like(ref[0])
            po.oracle().or_swiglu(ptr(ref[0]), ptr(ref[1]), ptr(sw), sw.size)
            d = np.abs(got.view(np.float16).astype(np.float32) - sw.view(np.float16).astype(np.float32))
            assert np.all(d <= np.abs(sw.view(np.float16).astype(np.float32)) * 2 ** -10 + 1e-7), (lo, hi)
            assert (got == sw).mean() > 0.99
    finally:
        L.ifr_linear_free(dev.ctx, dl)
        for b in (qd, sd, gd, od):
            b.free()
