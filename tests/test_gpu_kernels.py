"""Kernel-level parity of the gfx950 kernels against the CPU oracle (same seeded inputs).

Bit-exact: int32 T accumulators, the fp16 GEMM outputs (same fold order),
act-quant codes/scales/group sums, the packing maps.  Tolerance: attention
(fp16 P in the PV MFMA, online softmax), SwiGLU (device expf).
"""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import workloads as wl
from oracle import pyoracle as po
from oracle.pyoracle import ptr
from tests.conftest import announce

pytestmark = pytest.mark.gpu

L = ia.lib()

CFG2 = [("qkv", 1024, 4096), ("o", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)]
MS = [1, 8, 16, 64, 256, 1024]


def _gemm_case(dev, lin, M, rng, dump=True):
    x = rng.standard_normal((M, lin.K), dtype=np.float32)
    q, s, g = po.act_quant(x)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
    try:
        qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(s[:, 0].copy()), dev.upload(g)
        od = dev.alloc(M * lin.N * 2)
        ng = lin.K // 128
        td = dev.alloc(M * lin.N * ng * 4) if dump else None
        announce(f"qgemm N={lin.N} K={lin.K} bits={lin.bits} M={M}")
        ia.check(L.ifr_quant_gemm(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p,
                                  td.p if dump else None), "ifr_quant_gemm")
        out = dev.download(od, np.uint16, (M, lin.N))
        T = dev.download(td, np.int32, (M, lin.N, ng)) if dump else None
        for b in (qd, sd, gd, od) + ((td,) if dump else ()):
            b.free()
    finally:
        L.ifr_linear_free(dev.ctx, dl)
    return q, s, out, T


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("name,K,N", CFG2)
def test_qgemm_cfg2_bitexact(dev, name, K, N, bits):
    rng = np.random.default_rng(1000 + K + N + bits)
    lin = ia.make_linear(N, K, bits, rng)
    for M in MS:
        q, s, out, T = _gemm_case(dev, lin, M, rng, dump=M <= 256)
        ref = po.qgemm(q, s[:, 0], lin)
        if T is not None:
            Tr, _ = po.qgemm_ts(q, lin)
            assert np.array_equal(T, Tr), f"{name} M={M}: int32 T differs"
        bad = np.argwhere(out != ref)
        assert bad.size == 0, (
            f"{name} M={M}: {len(bad)} fp16 outputs differ, first: " +
            ", ".join(f"({m},{n}) dev {out[m, n]:#06x} oracle {ref[m, n]:#06x}" for m, n in bad[:6]))


def test_qgemm_general_zero_and_int8(dev):
    rng = np.random.default_rng(77)
    for bits in (2, 8):
        zero = rng.uniform(0, (1 << bits) - 1, size=(512, 1024 // 128))
        lin = ia.make_linear(512, 1024, bits, rng, zero=zero)
        for M in (3, 100):
            q, s, out, T = _gemm_case(dev, lin, M, rng)
            Tr, _ = po.qgemm_ts(q, lin)
            assert np.array_equal(T, Tr)
            assert np.array_equal(out, po.qgemm(q, s[:, 0], lin))


@pytest.mark.parametrize("bits,post", [(2, 2.0 / 3.0), (4, 2.0 * 0.37 / 15.0), (8, 2.0 / 255.0)])
def test_qgemm_post_scale_bitexact(dev, bits, post):
    """A per-linear output factor (the .intfer form post = 2*alpha/C) folds
    into the row scale: y = fp16((ascale * post) * acc), bit-exact."""
    rng = np.random.default_rng(500 + bits)
    post = float(np.float32(post))
    lin = ia.make_linear(1024, 2048, bits, rng, post=post)
    for M in (1, 64, 300):
        q, s, out, T = _gemm_case(dev, lin, M, rng, dump=False)
        ref = po.qgemm(q, s[:, 0], lin)
        assert np.array_equal(out, ref), f"bits={bits} M={M}: {(out != ref).sum()} outputs differ"
        unit = po.qgemm(q, s[:, 0], ia.HostLinear(lin.N, lin.K, bits, lin.codes, lin.scale, lin.zero,
                                                  lin.values, 0.0))
        assert not np.array_equal(out, unit)  # the factor is applied


@pytest.mark.parametrize("M", [1, 16, 64, 200])
def test_qgemm_swiglu_pair(dev, M):
    rng = np.random.default_rng(300 + M)
    F, K = 3072, 1024
    gate, up = ia.make_linear(F, K, 2, rng), ia.make_linear(F, K, 2, rng)
    x = rng.standard_normal((M, K), dtype=np.float32)
    q, s, g = po.act_quant(x)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(gate.struct), C.byref(up.struct), C.byref(dl)),
             "pair")
    qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(s[:, 0].copy()), dev.upload(g)
    od = dev.alloc(M * F * 2)
    announce(f"swiglu gemm M={M}")
    ia.check(L.ifr_quant_gemm_swiglu(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p), "swiglu")
    out = dev.download(od, np.uint16, (M, F))
    L.ifr_linear_free(dev.ctx, dl)
    for b in (qd, sd, gd, od):
        b.free()
    gh, uh = po.qgemm(q, s[:, 0], gate), po.qgemm(q, s[:, 0], up)
    ref = np.empty_like(gh)
    po.oracle().or_swiglu(ptr(gh), ptr(uh), ptr(ref), gh.size)
    # fp16 result of silu(g)*u: device expf may differ from libm by an ulp
    d = np.abs(out.view(np.float16).astype(np.float32) - ref.view(np.float16).astype(np.float32))
    tol = np.abs(ref.view(np.float16).astype(np.float32)) * 2 ** -10 + 1e-7
    assert np.all(d <= tol), d.max()
    assert (out == ref).mean() > 0.99


@pytest.mark.parametrize("bits,zmode", [(2, "codebook"), (4, "codebook"), (8, "codebook"), (2, "general"),
                                        (4, "general")])
def test_qgemm_every_launch_shape_bitexact(dev, bits, zmode):
    """Every launch shape of the table gives the oracle's bits (plain), and
    the same bits as every other shape (SwiGLU pair); shapes that do not
    apply decline with IFR_EDECLINE.  Codebook zeros (C/2) run the
    two-operation fold, general fp16 zeros the three-operation one.  An
    output that is not 16-byte aligned takes the per-element stores instead
    of the 16-byte row chunks, with the same bits."""
    rng = np.random.default_rng(900 + bits)
    nv = L.ifr_quant_gemm_variants()
    assert nv >= 2
    for (N, K) in ((512, 1024), (256, 3072), (384, 2048)):
        zero = None if zmode == "codebook" else rng.uniform(0, (1 << bits) - 1, size=(N, K // 128))
        lin = ia.make_linear(N, K, bits, rng, zero=zero)
        gate, up = ia.make_linear(N, K, bits, rng, zero=zero), ia.make_linear(N, K, bits, rng, zero=zero)
        dl, dp = C.c_void_p(), C.c_void_p()
        ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
        ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(gate.struct), C.byref(up.struct),
                                          C.byref(dp)), "pair")
        try:
            for M in (1, 5, 16, 37, 130):
                x = rng.standard_normal((M, K), dtype=np.float32)
                q, sc, g = po.act_quant(x)
                qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(sc[:, 0].copy()), dev.upload(g)
                od = dev.alloc(M * N * 2 + 16)
                od2 = C.c_void_p(od.p.value + 2)  # 2-byte aligned only
                ref = po.qgemm(q, sc[:, 0], lin)
                pair_out, ran = None, 0
                for v in range(nv):
                    announce(f"qgemm variant {v} bits={bits} N={N} K={K} M={M}")
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc == ia.IFR_EDECLINE:
                        continue
                    ia.check(rc, f"variant {v}")
                    out = dev.download(od, np.uint16, (M, N))
                    assert np.array_equal(out, ref), f"variant {v} N={N} K={K} M={M}"
                    ia.check(L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od2, v), "unaligned")
                    raw = dev.download(od, np.uint16, (M * N + 8,))
                    assert np.array_equal(raw[1:1 + M * N].reshape(M, N), ref), f"unaligned variant {v}"
                    ran += 1
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dp, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc == ia.IFR_EDECLINE:
                        continue
                    ia.check(rc, f"pair variant {v}")
                    po_ = dev.download(od, np.uint16, (M, N))
                    if pair_out is None:
                        pair_out = po_
                    assert np.array_equal(po_, pair_out), f"pair variant {v} N={N} K={K} M={M}"
                assert ran >= 2
                for b in (qd, sd, gd, od):
                    b.free()
        finally:
            L.ifr_linear_free(dev.ctx, dl)
            L.ifr_linear_free(dev.ctx, dp)


def test_qgemm_xcd_grouped_order_bitexact(dev):
    """A weight set large enough for the XCD-grouped block order of the
    larger-M shapes (INT8, N = 4096, K = 8192: 4 MB of codes per XCD share):
    every launch shape, and the default, give the oracle's bits."""
    rng = np.random.default_rng(977)
    N, K, M = 4096, 8192, 40
    lin = ia.make_linear(N, K, 8, rng)
    dl = C.c_void_p()
    ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
    try:
        x = rng.standard_normal((M, K), dtype=np.float32)
        q, sc, g = po.act_quant(x)
        qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(sc[:, 0].copy()), dev.upload(g)
        od = dev.alloc(M * N * 2)
        ref = po.qgemm(q, sc[:, 0], lin)
        ran = 0
        for v in list(range(L.ifr_quant_gemm_variants())) + [-1]:
            announce(f"qgemm grouped order variant {v} N={N} K={K} M={M}")
            if v < 0:
                rc = L.ifr_quant_gemm(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, None)
            else:
                rc = L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, v)
            if rc == ia.IFR_EDECLINE:
                continue
            ia.check(rc, f"variant {v}")
            assert np.array_equal(dev.download(od, np.uint16, (M, N)), ref), f"variant {v}"
            ran += 1
        assert ran >= 5
        for b in (qd, sd, gd, od):
            b.free()
    finally:
        L.ifr_linear_free(dev.ctx, dl)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_decode_stream_large_k_bitexact(dev, bits):
    """The decode weight-stream shapes (variants 13-15: M <= 16, the whole K
    of a column tile per workgroup) at the 27B-class depths K = 5120 and
    17408 (136 groups, the deepest register ring), against the oracle's
    bits, for the plain linear and the SwiGLU pair."""
    rng = np.random.default_rng(950 + bits)
    for (N, K) in ((96, 5120), (64, 17408)):
        lin = ia.make_linear(N, K, bits, rng)
        gate, up = ia.make_linear(N, K, bits, rng), ia.make_linear(N, K, bits, rng)
        dl, dp = C.c_void_p(), C.c_void_p()
        ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
        ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(gate.struct), C.byref(up.struct),
                                          C.byref(dp)), "pair")
        try:
            for M in (1, 3, 16):
                x = rng.standard_normal((M, K), dtype=np.float32)
                q, sc, g = po.act_quant(x)
                qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(sc[:, 0].copy()), dev.upload(g)
                od = dev.alloc(M * N * 2)
                ref = po.qgemm(q, sc[:, 0], lin)
                ran = 0
                pair_ref = None
                for v in (13, 14, 15, 0):
                    announce(f"qgemm stream variant {v} bits={bits} N={N} K={K} M={M}")
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc != ia.IFR_EDECLINE:
                        ia.check(rc, f"variant {v}")
                        out = dev.download(od, np.uint16, (M, N))
                        assert np.array_equal(out, ref), f"variant {v} N={N} K={K} M={M}"
                        ran += 1
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dp, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc != ia.IFR_EDECLINE:
                        ia.check(rc, f"pair variant {v}")
                        po_ = dev.download(od, np.uint16, (M, N))
                        if pair_ref is None:
                            pair_ref = po_
                        assert np.array_equal(po_, pair_ref), f"pair variant {v} N={N} K={K} M={M}"
                # A also given row-major (ifr_quant_gemm_rows: the stream
                # stages its A rows from it at M <= 4): the same bits
                qr = dev.upload(np.ascontiguousarray(q))
                for v in (13, 14, 15, -1):
                    announce(f"qgemm rows variant {v} bits={bits} N={N} K={K} M={M}")
                    for lin_d, want in ((dl, ref), (dp, pair_ref)):
                        rc = L.ifr_quant_gemm_rows(dev.ctx, lin_d, qd.p, qr.p, sd.p, gd.p, M, od.p, v)
                        if rc == ia.IFR_EDECLINE:
                            continue
                        ia.check(rc, f"rows variant {v}")
                        if want is not None:
                            assert np.array_equal(dev.download(od, np.uint16, (M, N)), want), \
                                f"rows variant {v} N={N} K={K} M={M} pair={lin_d is dp}"
                qr.free()
                # the heuristic's own choice (a stream shape, or its fallback
                # where one cannot hold the codes) gives the same bits
                ia.check(L.ifr_quant_gemm(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, None), "default")
                assert np.array_equal(dev.download(od, np.uint16, (M, N)), ref)
                ia.check(L.ifr_quant_gemm_swiglu(dev.ctx, dp, qd.p, sd.p, gd.p, M, od.p), "pair default")
                if pair_ref is not None:
                    assert np.array_equal(dev.download(od, np.uint16, (M, N)), pair_ref)
                assert ran >= (1 if bits < 8 else 0)
                for b in (qd, sd, gd, od):
                    b.free()
        finally:
            L.ifr_linear_free(dev.ctx, dl)
            L.ifr_linear_free(dev.ctx, dp)


@pytest.mark.parametrize("K,norm,rot,rnd,ga", [(1024, 1, 1, 0, 0), (1024, 0, 0, 1, 64),
                                               (2048, 0, 0, 0, 0), (3072, 1, 0, 0, 0),
                                               (5120, 1, 1, 0, 0)])
def test_act_quant_bitexact(dev, K, norm, rot, rnd, ga):
    rng = np.random.default_rng(K + 7 * norm + 3 * rot + ga)
    M = 37
    x = (rng.standard_normal((M, K), dtype=np.float32) * 2.5).astype(np.float32)
    x[5] = 0.0
    w = rng.normal(0, 0.1, size=K).astype(np.float32)
    q, s, g = po.act_quant(x, norm_w=w if norm else None, rotate=rot, round=rnd, ga=ga)
    ns = K // ga if ga else 1
    xd, wd = dev.upload(x), dev.upload(w)
    Mp = (M + 15) // 16 * 16
    qd, sd, gd = dev.alloc(Mp * K), dev.alloc(M * ns * 4), dev.alloc(M * (K // 128) * 4)
    announce(f"act_quant K={K} norm={norm} rot={rot} rnd={rnd} ga={ga}")
    ia.check(L.ifr_act_quant(dev.ctx, xd.p, M, K, wd.p if norm else None, C.c_float(1e-6), rot, rnd,
                             ga, qd.p, sd.p, gd.p), "ifr_act_quant")
    qg = ia.untile(dev.download(qd, np.int8, (Mp * K,)), M, K)
    sg = dev.download(sd, np.float32, (M, ns))
    gg = dev.download(gd, np.float32, (M, K // 128))
    for b in (xd, wd, qd, sd, gd):
        b.free()
    assert np.array_equal(qg, q)
    assert np.array_equal(sg.view(np.uint32), s.view(np.uint32))
    assert np.array_equal(gg, g)


def _attn_engine(dev, kv_int8, lens, chunks, dense_attention=0, model=None, max_rows=1200):
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = model or ia.SynthModel(cfg, seed=5)
    total = sum(lens) + sum(o + n for o, n in chunks)
    eng = ia.Engine(dev, model, max_seqs=len(lens) + len(chunks) + 1, max_seq_tokens=8192,
                    pool_tokens=total + 64 * (len(lens) + 4), kv_int8=kv_int8, max_rows=max_rows,
                    dense_attention=dense_attention)
    return cfg, model, eng


def test_chunked_region_matches_dense_units(dev):
    """The chunked region (4 q-blocks of a prefill chunk per workgroup, each
    K/V page staged once in LDS for all of them) gives the same bits as
    running every unit on its own: decode rows, full and ragged chunk groups
    (idle waves), chunks from offset 0 and at long offsets (up to 15 KV
    splits)."""
    lens = wl.cfg3_lengths(seed=3)[:24]
    chunks = [(0, 512), (1536, 200), (100, 37), (3500, 300), (31, 9), (7000, 64)]
    rng = np.random.default_rng(44)
    cfg = ia.default_cfg(layers=1, vocab=1024)
    nkv, hd, nq = cfg.n_kv, cfg.head_dim, cfg.n_heads
    all_lens = lens + [o + n for o, n in chunks]
    kvs = [(rng.standard_normal((1, n, nkv, hd), dtype=np.float32),
            rng.standard_normal((1, n, nkv, hd), dtype=np.float32)) for n in all_lens]
    outs, model = [], None
    for dense in (0, 1):
        cfg, model, eng = _attn_engine(dev, 0, lens, chunks, dense_attention=dense, model=model)
        seqs = []
        for k, v in kvs:
            s = eng.seq_open()
            eng.load_kv(s, k, v)
            seqs.append(s)
        rows = [(seqs[i], n - 1, 0, 0, 1) for i, n in enumerate(lens)]
        for j, (o, n) in enumerate(chunks):
            rows += [(seqs[len(lens) + j], o + p, 0, 1, 1) for p in range(n)]
        q = np.random.default_rng(45).standard_normal((len(rows), nq, hd), dtype=np.float32).astype(np.float16)
        announce(f"attention chunked region vs dense units: dense_attention={dense} M={len(rows)}")
        outs.append(eng.attention(0, rows, q))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_attention_cfg3(dev, kv_int8):
    lens = wl.cfg3_lengths(seed=3)
    chunks = [(0, 512), (1536, 512)]
    cfg, model, eng = _attn_engine(dev, kv_int8, lens, chunks)
    rng = np.random.default_rng(33)
    nkv, hd, nq = cfg.n_kv, cfg.head_dim, cfg.n_heads
    seqs, stored = [], []
    all_lens = lens + [o + n for o, n in chunks]
    for n in all_lens:
        s = eng.seq_open()
        k = rng.standard_normal((1, n, nkv, hd), dtype=np.float32)
        v = rng.standard_normal((1, n, nkv, hd), dtype=np.float32)
        eng.load_kv(s, k, v)
        # the stored values: fp16 round (then int8 per token/head)
        kr = k.astype(np.float16).astype(np.float32).reshape(n, nkv * hd)
        vr = v.astype(np.float16).astype(np.float32).reshape(n, nkv * hd)
        if kv_int8:
            for arr in (kr, vr):
                for t in range(n):
                    for h in range(nkv):
                        seg = np.ascontiguousarray(arr[t, h * hd:(h + 1) * hd])
                        po.oracle().or_kv_int8_round(ptr(seg), hd)
                        arr[t, h * hd:(h + 1) * hd] = seg
        seqs.append(s)
        stored.append((kr, vr))
    rows = [(seqs[i], n - 1, 0, 0, 1) for i, n in enumerate(lens)]
    for j, (o, n) in enumerate(chunks):
        rows += [(seqs[len(lens) + j], o + p, 0, 1, 1) for p in range(n)]
    M = len(rows)
    q = rng.standard_normal((M, nq, hd), dtype=np.float32).astype(np.float16)
    announce(f"attention cfg3 kv_int8={kv_int8} M={M}")
    out = eng.attention(0, rows, q)
    qf = q.astype(np.float32).reshape(M, nq * hd)
    sidx = {s: i for i, s in enumerate(seqs)}

    def ref_row(m):
        s, pos = rows[m][0], rows[m][1]
        kr, vr = stored[sidx[s]]
        o = np.empty(nq * hd, np.float32)
        po.oracle().or_attention_row(ptr(np.ascontiguousarray(qf[m])), ptr(np.ascontiguousarray(kr[:pos + 1])),
                                     ptr(np.ascontiguousarray(vr[:pos + 1])), pos, nq, nkv, hd, ptr(o))
        return o

    with ThreadPoolExecutor(8) as ex:
        ref = np.stack(list(ex.map(ref_row, range(M))))
    err = np.abs(out - ref)
    # fp16 probabilities in the PV product: |err| <= 4e-3 (values ~N(0,1) averages)
    assert err.max() < 4e-3, err.max()
    assert np.sqrt((err ** 2).mean()) < 5e-4


# (sequence lengths, rows as (sequence index, position, kind, want)):
# decode, verify and a 3-q-block chunk in one quad; then several quads of a
# chunk whose q-blocks span 3-4 KV splits, and a chunk that crosses a split
# boundary inside a quad (q-blocks of one quad with different split counts);
# then a cfg5-sized batch (a 2048-row chunk at offset 1000, decode, a verify
# group, a 700-row chunk from offset 0: M = 2754, so the pack kernel's
# threads hold up to three rows each)
PACK_CASES = [
    ([300, 40, 1000, 20],
     [(0, 299, 0, 1), (1, 30, 2, 1), (1, 31, 2, 1), (1, 32, 2, 1), (2, 999, 0, 0)] +
     [(3, p, 1, int(p == 19)) for p in range(20)]),
    ([513, 900, 64, 280],
     [(0, 512, 0, 1)] + [(1, 700 + p, 1, int(p == 199)) for p in range(200)] + [(2, 63, 0, 1)] +
     [(3, 240 + p, 1, int(p == 39)) for p in range(40)]),
    ([3100, 50, 2600, 700],
     [(0, 1000 + p, 1, int(p == 2047)) for p in range(2048)] + [(1, 49, 0, 1)] +
     [(2, 2590 + p, 2, 1) for p in range(5)] + [(3, p, 1, int(p == 699)) for p in range(700)]),
]


@pytest.mark.parametrize("case", range(len(PACK_CASES)))
def test_pack_maps_match_restatement(dev, case):
    from oracle import pack as pk
    lens, spec = PACK_CASES[case]
    cfg, model, eng = _attn_engine(dev, 0, lens, [], max_rows=max(1200, len(spec)))
    rng = np.random.default_rng(9)
    seqs = []
    for n in lens:
        s = eng.seq_open()
        k = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
        eng.load_kv(s, k, k)
        seqs.append(s)
    rows = [(seqs[i], pos, 0, kind, want) for i, pos, kind, want in spec]
    q = np.zeros((len(rows), cfg.n_heads, cfg.head_dim), np.float16)
    announce(f"pack maps case {case}: M={len(rows)}")
    eng.attention(0, rows, q)
    M = len(rows)
    cu = np.zeros(M + 1, np.int32)
    grp, cb, cn, ct = (np.zeros(M, np.int32) for _ in range(4))
    units = np.zeros(65536 * 8, np.int32)
    nu, split = C.c_int32(), C.c_int32()
    ia.check(L.ifr_debug_pack(eng.dev.ctx, M, ptr(cu), ptr(grp), ptr(cb), ptr(cn), ptr(ct),
                              ptr(units), C.byref(nu), C.byref(split)), "debug_pack")
    qb = 16 // (cfg.n_heads // cfg.n_kv)  # one 16-column MFMA tile of (token, head) per unit
    exp = pk.pack(rows, cfg.n_kv, qb, split.value)
    ng = len(exp["cu_seqlens"]) - 1
    assert cu[:ng + 1].tolist() == exp["cu_seqlens"]
    assert grp.tolist() == exp["row_grp"]
    assert cb.tolist() == exp["comb_base"] and cn.tolist() == exp["comb_nsplit"]
    assert ct.tolist() == exp["comb_tok"]
    assert nu.value == len(exp["units"])
    assert units[:8 * nu.value].reshape(-1, 8).tolist() == exp["units"]
    ns = C.c_int32()
    order = np.zeros(4 * 65536, np.int32)
    ia.check(L.ifr_debug_attn_order(eng.dev.ctx, ptr(order), order.size, C.byref(ns)), "order")
    assert order[:ns.value].tolist() == exp["order"]
    # every unit is dispatched exactly once
    live = sorted(u for u in exp["order"] if u >= 0)
    assert live == list(range(nu.value))
