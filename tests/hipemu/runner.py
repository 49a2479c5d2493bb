"""Run library scenarios on the CPU emulation (test infrastructure only).

Usage (the ASan runtime must be preloaded, which run_scenarios() does):
    python tests/hipemu/runner.py <scenario> [...]
Each scenario drives the same C-ABI calls as a GPU test, against the
emulated library, and checks the results against the CPU oracle where the
GPU test does.  Any out-of-bounds access aborts with an ASan report.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

SCENARIOS = {}


def scenario(f):
    SCENARIOS[f.__name__] = f
    return f


def use_emulated_library():
    """Point intfer_amd's ctypes table at the emulated library."""
    from intfer_amd import _abi
    from tests.hipemu import build as eb
    L = C.CDLL(str(eb.LIB))
    for name, (res, args) in _abi._PROTOS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _abi._lib = L
    return L


def say(msg):
    sys.stdout.write(f"[emu] {msg}\n")
    sys.stdout.flush()


# ---- scenarios ---------------------------------------------------------------------

@scenario
def smoke():
    """__graft_entry__.smoke(): tiny model, M=20 prefill."""
    import __graft_entry__ as g
    g.smoke()


def _small_cfg(ia, **over):
    base = dict(hidden=256, layers=2, n_heads=4, n_kv=2, inter=384, vocab=512)
    base.update(over)
    return ia.default_cfg(**base)


@scenario
def noop():
    """The emulation loads and a context opens (environment check)."""
    import intfer_amd as ia
    ia.Device(0).close()


@scenario
def gemm_shapes():
    """Every launch shape at small K/N and ragged M, bit-exact vs the oracle."""
    _gemm_shapes((2, 4, 8), ((64, 128), (32, 256), (96, 384), (64, 1024), (32, 3072)))


@scenario
def gemm_small():
    """Every launch shape, INT2 and INT8, at K below and above 4 groups."""
    _gemm_shapes((2, 8), ((32, 256), (32, 1024)))


@scenario
def gemm_wide():
    """Block-sized N (full and partial column blocks), plain and SwiGLU pair."""
    _gemm_shapes((2, 4, 8), ((256, 256), (384, 1024)), Ms=(1, 70, 130), pair_check=True)


@scenario
def gemm_grouped():
    """Enough column blocks (N = 4096) for the XCD-grouped block order of the
    larger-M shapes, ragged M."""
    _gemm_shapes((2,), ((4096, 128),), Ms=(70, 130))


@scenario
def gemm_stream():
    """The decode weight-stream shapes at the 27B-class depths (K = 5120 and
    17408) and M = 1, 5, 16, INT2 and INT4."""
    _gemm_shapes((2, 4), ((32, 5120), (16, 17408)), Ms=(1, 5, 16), pair_check=True)


@scenario
def gemm_stream_rows():
    """The weight-stream shapes alone at every row count class: A staged in
    LDS (M = 1 .. 4), the partial last row quad (M = 6, 7) and two full
    quads (M = 8), INT2 / INT4 / INT8; each also with A given row-major
    (ifr_quant_gemm_rows)."""
    _gemm_shapes((2, 4, 8), ((32, 5120), (16, 17408)), Ms=(1, 2, 3, 4, 6, 7, 8), pair_check=True,
                 variants=(13, 14, 15), rows=True)


@scenario
def gemm_full():
    """The whole-K row-block shapes (A in LDS by the LDS DMA, every load at
    entry) at K of 8, 16 and 24 groups, ragged M across 16- and 32-row
    blocks, INT2 and INT4, plain and SwiGLU pair."""
    _gemm_shapes((2, 4), ((64, 1024), (128, 2048), (64, 3072)), Ms=(1, 17, 40, 70), pair_check=True,
                 variants=range(16, 21))


def _gemm_shapes(bits_list, shapes, Ms=(1, 17, 70), pair_check=False, variants=None, rows=False):
    import intfer_amd as ia
    from oracle import pyoracle as po
    L = ia.lib()
    dev = ia.Device(0)
    rng = np.random.default_rng(5)
    nv = L.ifr_quant_gemm_variants()
    # each shape with codebook zeros (C/2: the two-operation fold) and with
    # general fp16 zeros (the three-operation fold)
    for bits, (N, K), zmode in [(b, s, z) for b in bits_list for s in shapes for z in ("codebook", "general")]:
        if True:
            zero = None if zmode == "codebook" else rng.uniform(0, (1 << bits) - 1, size=(N, K // 128))
            lin = ia.make_linear(N, K, bits, rng, zero=zero)
            gate = ia.make_linear(N, K, bits, rng, zero=zero)
            up = ia.make_linear(N, K, bits, rng, zero=zero)
            dl, dp = C.c_void_p(), C.c_void_p()
            ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
            ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(gate.struct), C.byref(up.struct),
                                              C.byref(dp)), "pair")
            for M in Ms:
                x = rng.standard_normal((M, K), dtype=np.float32)
                q, sc, g = po.act_quant(x)
                qd, sd, gd = dev.upload(ia.atile(q)), dev.upload(sc[:, 0].copy()), dev.upload(g)
                od = dev.alloc(M * N * 2)
                ref = po.qgemm(q, sc[:, 0], lin)
                pair_ref = None
                ran = 0
                for v in (range(nv) if variants is None else variants):
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dl, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc == ia.IFR_EDECLINE:
                        continue
                    ia.check(rc, f"variant {v}")
                    ran += 1
                    out = dev.download(od, np.uint16, (M, N))
                    assert np.array_equal(out, ref), f"bits {bits} N {N} K {K} M {M} variant {v} {zmode}"
                    rc = L.ifr_quant_gemm_variant(dev.ctx, dp, qd.p, sd.p, gd.p, M, od.p, v)
                    if rc != ia.IFR_EDECLINE:
                        ia.check(rc, f"pair variant {v}")
                        if pair_check:
                            po_ = dev.download(od, np.uint16, (M, N))
                            if pair_ref is None:
                                pair_ref = po_
                            assert np.array_equal(po_, pair_ref), f"pair variant {v} N {N} K {K} M {M}"
                    if rows:  # A also row-major: the same bits
                        qr = dev.upload(np.ascontiguousarray(q))
                        ia.check(L.ifr_quant_gemm_rows(dev.ctx, dl, qd.p, qr.p, sd.p, gd.p, M, od.p, v), "rows")
                        assert np.array_equal(dev.download(od, np.uint16, (M, N)), ref), f"rows variant {v}"
                        rc = L.ifr_quant_gemm_rows(dev.ctx, dp, qd.p, qr.p, sd.p, gd.p, M, od.p, v)
                        if pair_check and pair_ref is not None and rc != ia.IFR_EDECLINE:
                            ia.check(rc, "pair rows")
                            assert np.array_equal(dev.download(od, np.uint16, (M, N)), pair_ref), \
                                f"pair rows variant {v}"
                        qr.free()
                for b in (qd, sd, gd, od):
                    b.free()
                # (a restricted variant list may hold no shape for wide codes)
                assert ran > 0 or variants is not None, f"no launch shape ran: bits {bits} N {N} K {K} M {M}"
                say(f"gemm bits={bits} N={N} K={K} M={M} zeros={zmode} ok ({ran} shapes)")
            L.ifr_linear_free(dev.ctx, dl)
            L.ifr_linear_free(dev.ctx, dp)
    dev.close()


def _forward_case(layers, kv_int8, steps, hidden=1024, n_heads=16, n_kv=8, inter=3072,
                  vocab=2048, bits=2, intfer_form=False, seed=11):
    import intfer_amd as ia
    from intfer_amd import workloads as wl
    from oracle import pyoracle as po
    cfg = ia.default_cfg(layers=layers, hidden=hidden, n_heads=n_heads, n_kv=n_kv, inter=inter,
                         vocab=vocab)
    model = ia.SynthModel(cfg, seed=seed, bits=bits, intfer_form=intfer_form)
    dev = ia.Device(0)
    w = wl.cfg1(cfg, seed=1)
    eng = ia.Engine(dev, model, max_seqs=8, max_seq_tokens=2048, pool_tokens=8 * 2048,
                    kv_int8=kv_int8, max_rows=128)
    ora = po.OracleEngine(model, kv_int8=kv_int8, mode=0, max_seqs=8)
    dec_e, dec_o = [], []
    for (k, v) in w.kv:
        s = eng.seq_open()
        eng.load_kv(s, k, v)
        dec_e.append(s)
        so = ora.seq_open()
        kr = k.astype(np.float16).astype(np.float32)
        vr = v.astype(np.float16).astype(np.float32)
        if kv_int8:
            for arr in (kr, vr):
                flat = arr.reshape(-1, cfg.head_dim)
                for i in range(flat.shape[0]):
                    seg = np.ascontiguousarray(flat[i])
                    po.oracle().or_kv_int8_round(po.ptr(seg), cfg.head_dim)
                    flat[i] = seg
        ora.set_kv(so, kr.reshape(cfg.layers, k.shape[1], -1), vr.reshape(cfg.layers, k.shape[1], -1))
        dec_o.append(so)
    pe, pq = eng.seq_open(), ora.seq_open()
    t0 = time.time()
    be, lg = eng.forward(wl.cfg1_rows(w, dec_e, pe), logits=True)
    bo, lo = ora.forward(wl.cfg1_rows(w, dec_o, pq), logits=True)
    err = float(np.abs(lg - lo).max() / lo.std())
    say(f"cfg1 layers={layers} kv_int8={kv_int8}: {time.time() - t0:.1f}s, tokens equal "
        f"{np.array_equal(be, bo)}, max|dlogit|/std {err:.3g}")
    want = [i for i, r in enumerate(wl.cfg1_rows(w, dec_e, pe)) if r[4]]
    seq_e, seq_o = dec_e + [pe], dec_o + [pq]
    pos = [n + 1 for n in w.contexts] + [len(w.pre_tokens)]
    tok = [int(bo[i]) for i in want]
    for step in range(steps):
        be2, lg2 = eng.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_e, pos, tok)], logits=True)
        bo2, lo2 = ora.forward([(s, p, t, 0, 1) for s, p, t in zip(seq_o, pos, tok)], logits=True)
        say(f"  step {step}: agree {int((be2 == bo2).sum())}/5, max|dlogit|/std "
            f"{float(np.abs(lg2 - lo2).max() / lo2.std()):.3g}")
        tok = [int(x) for x in bo2]
        pos = [p + 1 for p in pos]
    dev.close()
    model.close()
    return err


@scenario
def forward_one_layer():
    """test_one_layer_bit_exact at a 2048-token vocabulary."""
    _forward_case(1, 0, 2)


@scenario
def forward_kv8():
    """cfg1 with int8 KV and greedy steps (two layers)."""
    _forward_case(2, 1, 3)


@scenario
def forward_fp16():
    """cfg1 with fp16 KV and greedy steps (two layers)."""
    _forward_case(2, 0, 3)


@scenario
def forward_one_layer_full_vocab():
    """test_one_layer_bit_exact at its real shape (vocabulary 151936)."""
    _forward_case(1, 0, 1, vocab=151936)


@scenario
def forward_full_fp16():
    """test_cfg1_mixed_iteration_and_greedy64[0] at its real shape, 2 greedy steps."""
    _forward_case(28, 0, 2, vocab=151936)


@scenario
def forward_full_kv8():
    """test_cfg1_mixed_iteration_and_greedy64[1] at its real shape, 2 greedy steps."""
    _forward_case(28, 1, 2, vocab=151936)


@scenario
def sched_small():
    """Scheduler split/joint/solo and spec verify rows on a small model."""
    import intfer_amd as ia
    from intfer_amd import workloads as wl
    cfg = ia.default_cfg(layers=2, vocab=2048)
    model = ia.SynthModel(cfg, seed=3, bits=2)
    dev = ia.Device(0)
    eng = ia.Engine(dev, model, max_seqs=16, max_seq_tokens=1024, pool_tokens=16 * 1024, max_rows=256)
    prompts = wl.cfg4_requests(4, seed=8, vocab=cfg.vocab, lo=40, hi=150)
    streams = []
    for split in (0, 1):
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8, split_iter=split)
        ids = [sch.submit(p, 5) for p in prompts]
        for _ in range(200):
            if sch.step() == 0 and all(sch.result(i)[1] for i in ids):
                break
        streams.append([sch.result(i)[0] for i in ids])
        sch.close()
    assert streams[0] == streams[1], streams
    say("split == joint")
    rng = np.random.default_rng(5)
    base = rng.integers(0, cfg.vocab, size=30).astype(np.int32)
    pr = [np.concatenate([base, base, base[:7]]).astype(np.int32), base[:25].copy()]
    out = []
    for k in (0, 4):
        sch = ia.Scheduler(eng, chunk_m=64, live_cap=8, spec_k=k)
        ids = [sch.submit(p, 8) for p in pr]
        n = 0
        while not all(sch.result(i)[1] for i in ids) and n < 100:
            sch.step()
            n += 1
        out.append([sch.result(i)[0] for i in ids])
        sch.close()
    assert out[0] == out[1], out
    say("spec == plain")
    dev.close()
    model.close()


@scenario
def attention_ragged(heads=(16, 8)):
    """Joint ragged attention (decode rows of several lengths + two causal
    chunks, one at an offset), fp16 and int8 KV, vs the oracle row loop."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    from oracle.pyoracle import ptr
    for kv_int8 in (0, 1):
        cfg = ia.default_cfg(layers=1, vocab=1024, n_heads=heads[0], n_kv=heads[1])
        model = ia.SynthModel(cfg, seed=5)
        dev = ia.Device(0)
        lens = [40, 300, 257, 1000, 33]
        chunks = [(0, 70), (520, 45)]
        eng = ia.Engine(dev, model, max_seqs=16, max_seq_tokens=4096, pool_tokens=8192,
                        kv_int8=kv_int8, max_rows=256)
        rng = np.random.default_rng(33)
        nkv, hd, nq = cfg.n_kv, cfg.head_dim, cfg.n_heads
        seqs, stored = [], []
        for n in lens + [o + m for o, m in chunks]:
            s = eng.seq_open()
            k = rng.standard_normal((1, n, nkv, hd), dtype=np.float32)
            v = rng.standard_normal((1, n, nkv, hd), dtype=np.float32)
            eng.load_kv(s, k, v)
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
        for j, (o, m) in enumerate(chunks):
            rows += [(seqs[len(lens) + j], o + p, 0, 1, 1) for p in range(m)]
        M = len(rows)
        q = rng.standard_normal((M, nq, hd), dtype=np.float32).astype(np.float16)
        out = eng.attention(0, rows, q)
        qf = q.astype(np.float32).reshape(M, nq * hd)
        sidx = {s: i for i, s in enumerate(seqs)}
        err = 0.0
        for m in range(M):
            s, pos = rows[m][0], rows[m][1]
            kr, vr = stored[sidx[s]]
            o = np.empty(nq * hd, np.float32)
            po.oracle().or_attention_row(ptr(np.ascontiguousarray(qf[m])), ptr(np.ascontiguousarray(kr[:pos + 1])),
                                         ptr(np.ascontiguousarray(vr[:pos + 1])), pos, nq, nkv, hd, ptr(o))
            err = max(err, float(np.abs(out[m] - o).max()))
        say(f"attention kv_int8={kv_int8} M={M}: max err {err:.3g}")
        assert err < 4e-3
        dev.close()
        model.close()


@scenario
def noalloc_limits():
    """ifr_attention_noalloc at its row limit (512 rows) with ~3100 of its
    4096 attention units (a 32-token KV split makes many short units), twice
    (large, then small), against ifr_attention bit for bit: ASan bounds the
    whole scratch array, and a region of it overlapping another would change
    the results.  Then the two refusals: 513 rows, and more than 4096 units."""
    import intfer_amd as ia
    cfg = ia.default_cfg(layers=1, vocab=512, hidden=256, n_heads=4, n_kv=2, inter=256)
    model = ia.SynthModel(cfg, seed=6)
    dev = ia.Device(0)
    L = ia.lib()
    eng = ia.Engine(dev, model, max_seqs=20, max_seq_tokens=2048, pool_tokens=20 * 2048, max_rows=600,
                    attn_split=32)
    rng = np.random.default_rng(44)
    nkv, hd, nq = cfg.n_kv, cfg.head_dim, cfg.n_heads
    seqs = []
    for n in [1024] + [64] * 16 + [2048]:
        s = eng.seq_open()
        eng.load_kv(s, rng.standard_normal((1, n, nkv, hd), dtype=np.float32),
                    rng.standard_normal((1, n, nkv, hd), dtype=np.float32))
        seqs.append(s)

    def noalloc(rows, q):
        arr = ia.rows_array(rows)
        M = len(arr)
        qd = dev.upload(np.ascontiguousarray(q, dtype=np.float16))
        od = dev.alloc(M * nq * hd * 4)
        try:
            rc = L.ifr_attention_noalloc(dev.ctx, 0, arr, M, qd.p, od.p)
            return rc, (dev.download(od, np.float32, (M, nq * hd)) if rc == 0 else None)
        finally:
            qd.free()
            od.free()

    big = [(seqs[0], 528 + p, 0, 1, 1) for p in range(496)] + [(seqs[1 + i], 63, 0, 0, 1) for i in range(16)]
    small = [(seqs[0], 1000 + p, 0, 1, 1) for p in range(20)] + [(seqs[1 + i], 63, 0, 0, 1) for i in range(3)]
    for name, rows in (("512 rows", big), ("23 rows", small)):
        q = rng.standard_normal((len(rows), nq, hd), dtype=np.float32).astype(np.float16)
        rc, got = noalloc(rows, q)
        assert rc == 0, L.ifr_last_error()
        ref = eng.attention(0, rows, q)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
        say(f"noalloc {name}: bit-identical to ifr_attention")
    over = big + [(seqs[-1], 0, 0, 1, 1)]
    rc, _ = noalloc(over, np.zeros((len(over), nq, hd), np.float16))
    assert rc == ia.IFR_EINVAL and b"no-allocation limit" in L.ifr_last_error()
    many = [(seqs[-1], 1536 + p, 0, 1, 1) for p in range(512)]  # 64 q-blocks x 2 heads x 49..64 splits
    rc, _ = noalloc(many, np.zeros((512, nq, hd), np.float16))
    assert rc == ia.IFR_EINVAL and b"attention units" in L.ifr_last_error()
    say("noalloc refusals: 513 rows, > 4096 units")
    del eng
    dev.close()
    model.close()


@scenario
def forward_gqa5():
    """A layer of the 27B-class shape family at small width: 40 q / 8 kv
    heads (GQA group 5), hidden 1280 (non-power-of-two Hadamard), an FFN of
    17 groups, mixed INT2 / INT4 widths, int8 KV."""
    err = _forward_case(1, 1, 1, hidden=1280, n_heads=40, n_kv=8, inter=2176, vocab=512, bits=0)
    # attention is fp32-accurate, not bit-identical: an int8 activation code
    # flip moves a logit row by a few hundredths of its sigma; a wrong head
    # or group mapping moves it by whole sigmas
    assert err < 0.2, err


@scenario
def attention_ragged_g5():
    """The same with a GQA group of 5 (the 27B-class 40 q / 8 kv heads),
    whose q-block of 3 tokens fills 15 of the 16 MFMA columns."""
    attention_ragged(heads=(10, 2))


@scenario
def forward_fused_qk():
    """The QKV GEMM with the q/k norm + RoPE + KV append epilogue (M > 128,
    one head per workgroup) against the two separate passes: logits and the
    following decode step bit-identical, fp16 and int8 KV.  A model without
    q/k norm weights (qk_norm = 0) takes the same epilogue without the norm,
    bit-identical to the separate pass and token-equal to the oracle."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    dev = ia.Device(0)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, 2048, size=150).tolist()
    for qkn, kv8 in ((1, 0), (1, 1), (0, 0)):
        cfg = ia.default_cfg(layers=1, vocab=2048, qk_norm=qkn)
        model = ia.SynthModel(cfg, seed=6, bits=2)
        outs = []
        for sep in (0, 1):
            eng = ia.Engine(dev, model, max_seqs=4, max_seq_tokens=512, pool_tokens=4 * 512, kv_int8=kv8,
                            max_rows=192, separate_qk=sep)
            s = eng.seq_open()
            eng.set_timing(True)
            b, lg = eng.forward([(s, p, t, ia.ROW_PREFILL, int(p % 50 == 49)) for p, t in enumerate(prompt)],
                                logits=True)
            # the 150-row forward ran the separate q/k pass only when asked to
            assert (eng.timing("qk_rope_kv")[1] > 0) == bool(sep), (sep, eng.timing("qk_rope_kv"))
            eng.set_timing(False)
            _, lg2 = eng.forward([(s, 150, int(b[-1]), ia.ROW_DECODE, 1)], logits=True)
            outs.append((lg, lg2, b))
            del eng
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1]), kv8
        if not qkn:
            ora = po.OracleEngine(model, kv_int8=kv8, mode=0, max_seqs=4)
            so = ora.seq_open()
            bo, lo = ora.forward([(so, p, t, ia.ROW_PREFILL, int(p % 50 == 49)) for p, t in enumerate(prompt)],
                                 logits=True)
            assert np.array_equal(bo, outs[0][2]), (bo, outs[0][2])
            assert float(np.abs(outs[0][0] - lo).max()) <= 0.05 * float(lo.std())
        say(f"fused q/k epilogue qk_norm={qkn} kv_int8={kv8}: logits and next step bit-identical to the two passes")
        model.close()
    dev.close()


@scenario
def gemm_f16():
    """The FP16-activation dequant GEMM (both kernels: M == 1 and tiled) in
    bounds and bit-exact against the oracle, INT2 / INT4 / INT8."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    L = ia.lib()
    dev = ia.Device(0)
    rng = np.random.default_rng(17)
    for bits in (2, 4, 8):
        N, K = 80, 256
        lin = ia.make_linear(N, K, bits, rng)
        dl = C.c_void_p()
        ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
        for M in (1, 3, 70):
            a = (rng.standard_normal((M, K)) * 2).astype(np.float16)
            ad, od = dev.upload(a.view(np.uint16)), dev.alloc(M * N * 2)
            ia.check(L.ifr_quant_gemm_f16(dev.ctx, dl, ad.p, M, C.c_float(0.5), od.p), "f16")
            got = dev.download(od, np.uint16, (M, N))
            ref = np.empty((M, N), np.uint16)
            po.oracle().or_qgemm_f16(po.ptr(a.view(np.uint16)), M, C.byref(lin.struct), np.float32(0.5),
                                     po.ptr(ref))
            assert np.array_equal(got, ref), (bits, M)
            ad.free()
            od.free()
        L.ifr_linear_free(dev.ctx, dl)
        say(f"fp16 GEMM bits={bits}: M = 1, 3, 70 bit-exact")
    dev.close()


@scenario
def gemm_ga():
    """The grouped-activation GEMM in bounds and bit-exact against the
    oracle, INT2 / INT4 / INT8, ga = 64 and K, ragged M."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    L = ia.lib()
    dev = ia.Device(0)
    rng = np.random.default_rng(19)
    for bits in (2, 4, 8):
        N, K = 80, 256
        lin = ia.make_linear(N, K, bits, rng)
        dl = C.c_void_p()
        ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(dl)), "upload")
        for M, ga in ((1, 64), (21, 0)):
            g = ga or K
            a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            asc = (rng.random((M, K // g)) * 0.05 + 1e-4).astype(np.float32)
            ad, sd, od = dev.upload(ia.atile(a)), dev.upload(asc), dev.alloc(M * N * 2)
            ia.check(L.ifr_quant_gemm_ga(dev.ctx, dl, ad.p, sd.p, M, ga, C.c_float(0.5), od.p), "ga")
            got = dev.download(od, np.uint16, (M, N))
            ref = np.empty((M, N), np.uint16)
            po.oracle().or_qgemm_ga(po.ptr(a), po.ptr(asc), M, g, C.byref(lin.struct), np.float32(0.5),
                                    po.ptr(ref))
            assert np.array_equal(got, ref), (bits, M, ga)
            for b in (ad, sd, od):
                b.free()
        L.ifr_linear_free(dev.ctx, dl)
        say(f"grouped-activation GEMM bits={bits}: M = 1, 21 bit-exact")
    dev.close()


@scenario
def forward_gated():
    """The attention output gate: a gated one-layer model through the fused
    QKV epilogue (150 prefill rows) and the separate q/k pass (the decode
    row, and a separate_qk engine): fused == separate bit for bit, tokens
    equal to the oracle's; and zero gate rows (sigmoid = 1/2) give the
    ungated model with its O projection halved, bit for bit."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    dev = ia.Device(0)
    rng = np.random.default_rng(13)
    prompt = rng.integers(0, 2048, size=150).tolist()

    def run(model, sep):
        eng = ia.Engine(dev, model, max_seqs=4, max_seq_tokens=512, pool_tokens=4 * 512, max_rows=192,
                        separate_qk=sep)
        s = eng.seq_open()
        b, lg = eng.forward([(s, p, t, ia.ROW_PREFILL, int(p % 50 == 49)) for p, t in enumerate(prompt)],
                            logits=True)
        _, lg2 = eng.forward([(s, 150, int(b[-1]), ia.ROW_DECODE, 1)], logits=True)
        del eng
        return b, lg, lg2

    cfg = ia.default_cfg(layers=1, vocab=2048, attn_gate=1)
    model = ia.SynthModel(cfg, seed=6, bits=2)
    outs = [run(model, sep) for sep in (0, 1)]
    assert all(np.array_equal(outs[0][i], outs[1][i]) for i in range(3))
    ora = po.OracleEngine(model, mode=0, max_seqs=4)
    so = ora.seq_open()
    bo, lo = ora.forward([(so, p, t, ia.ROW_PREFILL, int(p % 50 == 49)) for p, t in enumerate(prompt)], logits=True)
    assert np.array_equal(bo, outs[0][0]), (bo, outs[0][0])
    err = float(np.abs(outs[0][1] - lo).max() / lo.std())
    assert err <= 0.05, err
    say(f"gated forward: fused == separate, tokens equal to the oracle, max|dlogit|/std {err:.3g}")
    model.close()
    gated = ia.SynthModel(cfg, seed=6, bits=2)
    plain = ia.SynthModel(ia.default_cfg(layers=1, vocab=2048), seed=6, bits=2)
    q = gated.layer(0).q
    sc = np.ctypeslib.as_array(q.scale, shape=(q.N, q.K // 128))
    for h in range(cfg.n_heads):
        sc[(2 * h + 1) * 128:(2 * h + 2) * 128] = 0
    plain.ptr.contents.layers[0].o.post = 0.5
    a, b = run(gated, 0), run(plain, 0)
    assert all(np.array_equal(a[i], b[i]) for i in range(3))
    say("zero gate == ungated with the O projection halved, bit for bit")
    gated.close()
    plain.close()
    dev.close()


@scenario
def prefix_copy():
    """ifr_seq_copy_prefix (the prefix cache's page copy) with fp16 and int8
    KV: a copied prefix plus the recomputed rest gives the same logits, bit
    for bit, as the sequence it was copied from; then the scheduler's cache
    reproduces the uncached streams of two chat turns."""
    import intfer_amd as ia
    cfg = _small_cfg(ia, layers=2)
    model = ia.SynthModel(cfg, seed=5, bits=2)
    dev = ia.Device(0)
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, cfg.vocab, size=70).tolist()
    for kv8 in (0, 1):
        eng = ia.Engine(dev, model, max_seqs=4, max_seq_tokens=256, pool_tokens=4 * 256,
                        kv_int8=kv8, max_rows=96)
        a = eng.seq_open()
        ba, la = eng.forward([(a, p, t, ia.ROW_PREFILL, int(p == 69)) for p, t in enumerate(prompt)],
                             logits=True)
        for cut in (45, 64, 1):
            b = eng.seq_open()
            eng.seq_copy_prefix(b, a, cut)
            bb, lb = eng.forward([(b, p, prompt[p], ia.ROW_PREFILL, int(p == 69))
                                  for p in range(cut, 70)], logits=True)
            assert np.array_equal(la, lb), (kv8, cut, float(np.abs(la - lb).max()))
            # and one decode step on both
            t = int(ba[-1])
            _, da = eng.forward([(a, 70, t, ia.ROW_DECODE, 1)], logits=True)
            _, db = eng.forward([(b, 70, t, ia.ROW_DECODE, 1)], logits=True)
            assert np.array_equal(da, db), (kv8, cut)
            eng.seq_truncate(a, 70)
            eng.seq_close(b)
        say(f"copy prefix kv_int8={kv8}: logits bit-identical at cuts 45, 64, 1")
        p2 = prompt[:50]
        outs = []
        for n in (0, 2):
            sch = ia.Scheduler(eng, chunk_m=32, live_cap=4, prefix_cache=n)
            g1 = _drive(sch, p2, 3)
            g2 = _drive(sch, p2 + g1 + prompt[50:60], 3)
            outs.append((g1, g2))
            sch.close()
        assert outs[0] == outs[1], outs
        say(f"scheduler prefix cache kv_int8={kv8}: streams equal")
        eng.seq_close(a)
    dev.close()
    model.close()


def _drive(sch, prompt, max_new):
    rid = sch.submit(prompt, max_new)
    for _ in range(200):
        if sch.step() == 0 and sch.result(rid)[1]:
            break
    out, done = sch.result(rid)
    assert done
    return out


@scenario
def act_quant():
    import intfer_amd as ia
    from oracle import pyoracle as po
    L = ia.lib()
    dev = ia.Device(0)
    # 1024 has its own kernel; the register kernel takes every K whose tail
    # per thread is 0 or a power of two (P = floor_pow2(K)): 256, 512, 768,
    # 1280, 2048, 2304, 3072, 5120, 6144, 8192; 1792 (tail 3) takes the LDS one
    for (K, norm, rot, rnd, ga) in [(1024, 1, 1, 0, 0), (1024, 0, 0, 1, 64), (2048, 0, 0, 0, 0),
                                    (3072, 1, 0, 0, 0), (5120, 1, 1, 0, 0), (256, 1, 1, 0, 0),
                                    (512, 1, 1, 0, 64), (768, 1, 1, 0, 0), (1280, 1, 1, 1, 64),
                                    (2304, 1, 1, 0, 0), (5120, 1, 1, 1, 64), (6144, 1, 1, 0, 0),
                                    (8192, 0, 1, 0, 64), (1792, 1, 1, 0, 0)]:
        rng = np.random.default_rng(K)
        M = 19
        x = (rng.standard_normal((M, K), dtype=np.float32) * 2.5).astype(np.float32)
        w = rng.normal(0, 0.1, size=K).astype(np.float32)
        q, s, g = po.act_quant(x, norm_w=w if norm else None, rotate=rot, round=rnd, ga=ga)
        ns = K // ga if ga else 1
        xd, wd = dev.upload(x), dev.upload(w)
        Mp = (M + 15) // 16 * 16
        qd, sd, gd = dev.alloc(Mp * K), dev.alloc(M * ns * 4), dev.alloc(M * (K // 128) * 4)
        ia.check(L.ifr_act_quant(dev.ctx, xd.p, M, K, wd.p if norm else None, C.c_float(1e-6), rot, rnd,
                                 ga, qd.p, sd.p, gd.p), "ifr_act_quant")
        qg = ia.untile(dev.download(qd, np.int8, (Mp * K,)), M, K)
        assert np.array_equal(qg, q), K
        assert np.array_equal(dev.download(sd, np.float32, (M, ns)).view(np.uint32), s.view(np.uint32)), K
        assert np.array_equal(dev.download(gd, np.float32, (M, K // 128)), g), K
        say(f"act_quant K={K} norm={norm} rot={rot} round={rnd} ga={ga} ok")
    dev.close()


@scenario
def intfer_load():
    """An .intfer image (container-form model, post = 2/C, mixed widths)
    loaded through ifr_model_load_intfer runs one prefill chunk like the
    oracle; then truncated / corrupted images through the parser and the
    host-model mapping, every access bounds-checked."""
    import intfer_amd as ia
    from oracle import pyoracle as po
    cfg = _small_cfg(ia, layers=1, n_heads=2, n_kv=1)
    model = ia.SynthModel(cfg, seed=5, bits=0, intfer_form=True)
    blob = model.write_intfer("emu")
    dev = ia.Device(0)
    eng = ia.Engine(dev, cfg, max_seqs=2, max_seq_tokens=256, max_rows=64, intfer=blob)
    ora = po.OracleEngine(model, kv_int8=0, mode=0, max_seqs=2)
    se, so = eng.seq_open(), ora.seq_open()
    rows = [(p, 7 + 3 * p) for p in range(20)]
    be, lg = eng.forward([(se, p, t, 1, 1) for p, t in rows], logits=True)
    bo, lo = ora.forward([(so, p, t, 1, 1) for p, t in rows], logits=True)
    err = float(np.abs(lg - lo).max() / lo.std())
    say(f"intfer forward: tokens equal {np.array_equal(be, bo)}, max|dlogit|/std {err:.3g}")
    assert np.array_equal(be, bo) and err < 2e-3
    rng = np.random.default_rng(1)
    js_len = int.from_bytes(blob[46:54], "little")
    n_err = 0
    for trial in range(60):
        img = bytearray(blob[:54 + js_len + 4096]) if trial % 2 else bytearray(blob)
        if trial % 3 == 0:
            img = img[:int(rng.integers(0, len(img)))]
        else:
            for _ in range(int(rng.integers(1, 4))):
                img[int(rng.integers(0, 54 + js_len))] = int(rng.integers(0, 256))
        try:
            f = ia.IntferFile(bytes(img))
            f.host_model(cfg).close()
            f.close()
        except ia.IfrError:
            n_err += 1
    say(f"intfer parse fuzz: {n_err}/60 refused cleanly")
    dev.close()
    model.close()


def _child_env() -> dict:
    from tests.hipemu import build as eb
    env = dict(os.environ)
    pre = env.get("LD_PRELOAD", "")
    env["LD_PRELOAD"] = eb.asan_runtime() + (":" + pre if pre else "")
    env["IFR_EMU_CHILD"] = "1"
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=1:detect_stack_use_after_return=0"
    return env


def run_scenarios(names, timeout=3600) -> int:
    """Run scenarios in a child process with the ASan runtime preloaded."""
    r = subprocess.run([sys.executable, str(HERE / "runner.py"), *names], env=_child_env(), timeout=timeout)
    return r.returncode


class ScenarioPool:
    """Every scenario in a child process of its own, at most `jobs` at once,
    started in the given order as soon as a slot frees up; result() waits for
    the named ones.  close() kills the children it started (by their own
    process ids) that are still running."""

    def __init__(self, names, jobs):
        import threading
        self._env = _child_env()
        self._todo = list(names)
        self._jobs = max(1, jobs)
        self._procs = {}
        self._rc = {}
        self._cv = threading.Condition()
        self._closed = False
        self._thread = threading.Thread(target=self._loop, daemon=True)
        self._thread.start()

    def _loop(self):
        while True:
            with self._cv:
                for n, p in list(self._procs.items()):
                    if p.poll() is not None:
                        self._rc[n] = p.returncode
                        del self._procs[n]
                        self._cv.notify_all()
                if self._closed or (not self._todo and not self._procs):
                    return
                while self._todo and len(self._procs) < self._jobs:
                    n = self._todo.pop(0)
                    self._procs[n] = subprocess.Popen([sys.executable, str(HERE / "runner.py"), n], env=self._env)
            time.sleep(0.2)

    def result(self, names, timeout=3600) -> int:
        end = time.time() + timeout
        with self._cv:
            while not all(n in self._rc for n in names):
                left = end - time.time()
                if left <= 0:
                    raise TimeoutError(f"scenarios {names} still running after {timeout} s")
                self._cv.wait(min(left, 1.0))
            return next((self._rc[n] for n in names if self._rc[n] != 0), 0)

    def close(self):
        with self._cv:
            self._closed = True
            for p in self._procs.values():
                p.kill()
            for p in self._procs.values():
                p.wait()
        self._thread.join()


if __name__ == "__main__":
    if os.environ.get("IFR_EMU_CHILD") != "1":
        sys.exit(run_scenarios(sys.argv[1:]))
    use_emulated_library()
    for n in sys.argv[1:]:
        say(f"scenario {n}")
        t = time.time()
        SCENARIOS[n]()
        say(f"scenario {n} passed in {time.time() - t:.1f}s")
