"""The FP16-activation dequant GEMM (ifr_quant_gemm_f16: the reference's
default GPU linear, quant_gemm_forward_usm, quant_gemm.cpp:359-2153) on the
device against the oracle's restatement, bit for bit: fp32 accumulation in
ascending k, w = (scale * alpha) * canonical codebook value, fp32 weights and
fused steps at M == 1, fp16-rounded weights at M > 1.  The oracle is pinned
in tests/test_oracle.py (numpy float32 step by step; exact rational fma)."""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr
from tests.conftest import announce

pytestmark = pytest.mark.gpu
L = ia.lib()


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("N,K", [(256, 1024), (144, 3072)])
def test_qgemm_f16_matches_oracle(dev, bits, N, K):
    rng = np.random.default_rng(bits * 7 + K)
    lin = ia.make_linear(N, K, bits, rng)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
    try:
        for M, alpha in ((1, 1.0), (1, 0.37), (3, 1.0), (64, 2.5), (130, 1.0)):
            a = (rng.standard_normal((M, K)) * 2).astype(np.float16)
            ad = dev.upload(a.view(np.uint16))
            od = dev.alloc(M * N * 2)
            announce(f"fp16 GEMM bits={bits} N={N} K={K} M={M}")
            ia.check(L.ifr_quant_gemm_f16(dev.ctx, dl, ad.p, M, C.c_float(alpha), od.p), "f16 gemm")
            got = dev.download(od, np.uint16, (M, N))
            ref = np.empty((M, N), np.uint16)
            po.oracle().or_qgemm_f16(ptr(a.view(np.uint16)), M, C.byref(lin.struct), np.float32(alpha), ptr(ref))
            assert np.array_equal(got, ref), (M, alpha)
            ad.free()
            od.free()
    finally:
        L.ifr_linear_free(dev.ctx, dl)


def test_qgemm_f16_declines_non_codebook_and_pairs(dev):
    rng = np.random.default_rng(3)
    N, K = 64, 256
    gen = ia.make_linear(N, K, 2, rng, zero=rng.uniform(0, 3, size=(N, K // 128)))
    g, u = ia.make_linear(N, K, 2, rng), ia.make_linear(N, K, 2, rng)
    d1, d2 = C.c_void_p(), C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(gen.struct), C.byref(d1)), "upload")
    ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(g.struct), C.byref(u.struct), C.byref(d2)), "pair")
    a = dev.alloc(4 * K * 2)
    o = dev.alloc(4 * N * 2 * 2)
    try:
        for d in (d1, d2):
            assert L.ifr_quant_gemm_f16(dev.ctx, d, a.p, 4, C.c_float(1.0), o.p) == ia.IFR_EDECLINE
    finally:
        L.ifr_linear_free(dev.ctx, d1)
        L.ifr_linear_free(dev.ctx, d2)
