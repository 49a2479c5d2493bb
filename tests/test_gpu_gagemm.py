"""The W2A8 / W4A8 / W8A8 GEMM with grouped activation scales
(ifr_quant_gemm_ga: the reference's DPAS fold as written, dpas48_tiled,
quant_gemm.cpp:3492-3791, per-op math :3602-3736, act_group :3502, :3614) on
the device against the oracle's restatement, bit for bit: per 32-wide K op,
acc += as(m, k0/ga) * ws * alpha * (2T - C S) * (1/C) in fp32, ops ascending.
The oracle is pinned in tests/test_oracle.py (one-hot slices and groups,
exact rational arithmetic per op, GA = K against equal slices, float64)."""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr
from tests.conftest import announce

pytestmark = pytest.mark.gpu
L = ia.lib()


def _ref(a, asc, M, ga, lin, alpha):
    ref = np.empty((M, lin.N), np.uint16)
    po.oracle().or_qgemm_ga(ptr(np.ascontiguousarray(a)), ptr(np.ascontiguousarray(asc, np.float32)), M, ga,
                            C.byref(lin.struct), np.float32(alpha), ptr(ref))
    return ref


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("N,K", [(256, 1024), (80, 3072)])
def test_qgemm_ga_matches_oracle(dev, bits, N, K):
    rng = np.random.default_rng(bits * 11 + K)
    lin = ia.make_linear(N, K, bits, rng)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
    try:
        for M, ga, alpha in ((1, 64, 1.0), (5, 64, 0.37), (16, 0, 1.0), (37, 128, 2.5), (130, 64, 1.0)):
            g = ga or K
            a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            asc = (rng.random((M, K // g)) * 0.05 + 1e-4).astype(np.float32)
            ad, sd = dev.upload(ia.atile(a)), dev.upload(asc)
            od = dev.alloc(M * N * 2)
            announce(f"grouped-activation GEMM bits={bits} N={N} K={K} M={M} ga={ga}")
            ia.check(L.ifr_quant_gemm_ga(dev.ctx, dl, ad.p, sd.p, M, ga, C.c_float(alpha), od.p), "ga gemm")
            got = dev.download(od, np.uint16, (M, N))
            assert np.array_equal(got, _ref(a, asc, M, g, lin, alpha)), (M, ga, alpha)
            for b in (ad, sd, od):
                b.free()
    finally:
        L.ifr_linear_free(dev.ctx, dl)


@pytest.mark.parametrize("bits", [2, 4])
def test_act_quant_ga64_then_gemm_matches_oracle(dev, bits):
    """The reference's W2A8 chain with its default act_group: the device
    act-quant (rotation, per-row 64-wide slices, half-away rounding) feeds the
    grouped-activation GEMM; the oracle runs its own act-quant and fold."""
    rng = np.random.default_rng(5 + bits)
    M, N, K = 23, 128, 1024
    lin = ia.make_linear(N, K, bits, rng)
    x = (rng.standard_normal((M, K), dtype=np.float32) * 1.7).astype(np.float32)
    q, s, _ = po.act_quant(x, rotate=1, round=0, ga=64)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
    Mp = (M + 15) // 16 * 16
    xd = dev.upload(x)
    qd, sd, gd, od = dev.alloc(Mp * K), dev.alloc(M * (K // 64) * 4), dev.alloc(M * (K // 128) * 4), dev.alloc(M * N * 2)
    try:
        announce(f"act_quant ga64 + grouped-activation GEMM bits={bits}")
        ia.check(L.ifr_act_quant(dev.ctx, xd.p, M, K, None, C.c_float(1e-6), 1, 0, 64, qd.p, sd.p, gd.p),
                 "ifr_act_quant")
        ia.check(L.ifr_quant_gemm_ga(dev.ctx, dl, qd.p, sd.p, M, 64, C.c_float(1.0), od.p), "ga gemm")
        got = dev.download(od, np.uint16, (M, N))
        assert np.array_equal(got, _ref(q, s, M, 64, lin, 1.0))
    finally:
        for b in (xd, qd, sd, gd, od):
            b.free()
        L.ifr_linear_free(dev.ctx, dl)


def test_qgemm_ga_declines_and_rejects(dev):
    rng = np.random.default_rng(3)
    N, K = 64, 256
    gen = ia.make_linear(N, K, 2, rng, zero=rng.uniform(0, 3, size=(N, K // 128)))
    cb = ia.make_linear(N, K, 2, rng)
    g, u = ia.make_linear(N, K, 2, rng), ia.make_linear(N, K, 2, rng)
    d1, d2, d3 = C.c_void_p(), C.c_void_p(), C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(gen.struct), C.byref(d1)), "upload")
    ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(g.struct), C.byref(u.struct), C.byref(d2)), "pair")
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(cb.struct), C.byref(d3)), "upload")
    a, s, o = dev.alloc(16 * K), dev.alloc(4 * K), dev.alloc(4 * N * 2 * 2)
    try:
        for d in (d1, d2):
            assert L.ifr_quant_gemm_ga(dev.ctx, d, a.p, s.p, 4, 64, C.c_float(1.0), o.p) == ia.IFR_EDECLINE
        for ga in (32, 96, -64):
            assert L.ifr_quant_gemm_ga(dev.ctx, d3, a.p, s.p, 4, ga, C.c_float(1.0), o.p) == ia.IFR_EINVAL
    finally:
        for b in (a, s, o):
            b.free()
        for d in (d1, d2, d3):
            L.ifr_linear_free(dev.ctx, d)
