"""Pins of the CPU oracle (oracle/oracle.cpp) before it is trusted as the checker.

Each oracle function is checked against something other than itself:
  or_f2h / or_h2f        reference dashq float_to_half / half_to_float (all 65536
                         halves + 2M float patterns) and numpy's IEEE conversion
  or_act_quant (GA64)    reference dashq::act_quant_ga64_batch, both roundings,
                         random rows and .5-tie-adversarial rows
  or_act_quant (per row) numpy float32 closed form of the same rule
  or_rot                 reference make_hadamard + apply_rotation_fwht (bit-exact,
                         pow2 and blockdiag(H_p, I)); dense H in float64
  or_dequant             reference QuantResult::dequant (canonical codebook)
  or_rmsnorm             float64 formula (1+w form, eps) -- order is checked
                         bit-exactly against the GPU kernel, not here
  or_qgemm_ts            int64 brute force
  or_qgemm (fold)        float64 dequant GEMM
  or_qgemm_f16           numpy float32 step by step (M > 1); exact rational
                         fma per step, the unfused form differing (M == 1);
                         float64 dequant GEMM
  or_qgemm_ga            one-hot activations naming the slice, group and code
                         used (exact powers of two); exact rational
                         arithmetic rounded per op (unit scales); GA = K
                         equal to GA = 64 with equal slices; float64 dequant
                         GEMM
  or_lmhead_quant        numpy float32 closed form of main.cpp:1745-1761
  or_lmhead / or_argmax  float64 logits; first-max-wins on planted ties
  or_attention_row       float64 softmax attention
  or_attention_row_split float64 softmax attention (page / split boundaries,
                         a moving running max); within last ulps of the loop
  or_rope                float64 cos/sin of the float32 angle
  forward (a8 / f32)     chunk invariance (M=1 == M=8 rows), f32 ~ a8 agreement
  forward (f32), whole   a float64 numpy restatement of the layer (norms,
                         rotation as the dense Hadamard, q/k norm, RoPE,
                         causal GQA attention, output gate, SwiGLU, tied
                         lm_head) from the model's own tensors: 1e-4 sigma
  output gate            zero gate rows == the ungated model with its O
                         projection halved, bit for bit, a8 and f32
Parity unpinned: none of the oracle functions above.
"""
import ctypes as C

import numpy as np
import pytest

import intfer_amd as ia
from oracle import pyoracle as po
from oracle.pyoracle import ptr

# The pin library is loaded only inside the tests that use it (po.ref()),
# so a run that deselects them (the GPU tests) never maps it.
HAVE_REF = po.REF_LIB.exists()
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built (no reference tree)")


@pytest.fixture(scope="module")
def O():
    return po.oracle()


# ---- fp16 --------------------------------------------------------------------------

def test_h2f_all_halves_match_reference_and_numpy(O):
    h = np.arange(65536, dtype=np.uint16)
    ours = np.empty(65536, np.float32)
    O.or_h2f_batch(ptr(h), ptr(ours), 65536)
    npv = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(npv)
    assert np.array_equal(ours.view(np.uint32)[fin], npv.view(np.uint32)[fin])
    assert np.all(np.isnan(ours[np.isnan(npv)]))
    if HAVE_REF:
        ref = np.array([po.ref().ref_half_to_float(int(x)) for x in h[::7]], np.float32)
        f7 = fin[::7]  # NaN payloads do not survive a Python float round trip
        assert np.array_equal(ours[::7].view(np.uint32)[f7], ref.view(np.uint32)[f7])


def test_f2h_matches_reference_and_numpy(O):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    # plus every half-way point between consecutive halves (RNE ties)
    h = np.arange(0, 0x7C00, dtype=np.uint32)
    lo = h.astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([bits.view(np.float32), mids, -mids]).astype(np.float32)
    x = x[np.isfinite(x)]
    ours = np.empty(x.size, np.uint16)
    O.or_f2h_batch(ptr(x), ptr(ours), x.size)
    with np.errstate(over="ignore"):
        npv = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, npv)
    if HAVE_REF:
        sub = x[::997]
        ref = np.array([po.ref().ref_float_to_half(float(v)) for v in sub], np.uint16)
        assert np.array_equal(ours[::997], ref)


# ---- act-quant ---------------------------------------------------------------------

def _tie_rows(rng, M, K):
    """Rows where many x*inv land exactly on .5 (half-away vs RNE differ)."""
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    for m in range(M):
        mx = np.float32(127.0)  # s = 1 -> inv = 1, x*inv = x
        x[m, :] = (rng.integers(-126, 126, size=K) + 0.5).astype(np.float32)
        x[m, 0] = mx
    return x


@needs_ref
@pytest.mark.parametrize("rnd", [0, 1])
def test_act_quant_ga64_matches_reference(O, rnd):
    rng = np.random.default_rng(2)
    K = 1024
    x = np.concatenate([rng.normal(0, 1, size=(8, K)).astype(np.float32) * 3,
                        _tie_rows(rng, 4, K),
                        np.zeros((1, K), np.float32)])
    q, s, _ = po.act_quant(x, round=rnd, ga=64)
    for m in range(x.shape[0]):
        qr = np.empty(K, np.int8)
        sr = np.empty(K // 64, np.float32)
        po.ref().ref_act_quant_ga64(ptr(x[m].copy()), ptr(qr), ptr(sr), K, rnd)
        assert np.array_equal(q[m], qr), f"row {m}"
        assert np.array_equal(s[m].view(np.uint32), sr.view(np.uint32))
    # the tie rows really exercise both roundings
    qa, _, _ = po.act_quant(x[8:12], round=0, ga=64)
    qb, _, _ = po.act_quant(x[8:12], round=1, ga=64)
    assert (qa != qb).sum() > 100


def _np_quant_row(x, rnd):
    x = x.astype(np.float32)
    mx = np.float32(max(np.float32(1e-6), np.abs(x).max()))
    s = np.float32(mx / np.float32(127.0))
    inv = np.float32(np.float32(1.0) / s)
    v = np.clip(x * inv, np.float32(-127), np.float32(127)).astype(np.float32)
    if rnd == 0:
        q = np.trunc((v + np.copysign(np.float32(0.5), v)).astype(np.float32))
    else:
        q = np.rint(v)
    return q.astype(np.int8), s


@pytest.mark.parametrize("rnd", [0, 1])
def test_act_quant_per_token_closed_form(O, rnd):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 2, size=(6, 2048)).astype(np.float32),
                        _tie_rows(rng, 2, 2048), np.zeros((1, 2048), np.float32)])
    q, s, g = po.act_quant(x, round=rnd, ga=0)
    for m in range(x.shape[0]):
        qe, se = _np_quant_row(x[m], rnd)
        assert np.array_equal(q[m], qe)
        assert s[m, 0] == se
        assert np.array_equal(g[m], q[m].astype(np.int64).reshape(-1, 128).sum(1).astype(np.float32))


# ---- rotation ------------------------------------------------------------------------

@pytest.mark.parametrize("dim", [128, 1024, 4096, 5120])
def test_rotation_matches_reference_and_dense(O, dim):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, size=dim).astype(np.float32)
    out = np.empty(dim, np.float32)
    O.or_rot(ptr(x), ptr(out), dim)
    if HAVE_REF:
        ro = np.empty(dim, np.float32)
        mat = np.empty(dim * dim, np.float32) if dim <= 1024 else None
        assert po.ref().ref_rotation_fwht(dim, ptr(x), ptr(ro), ptr(mat) if mat is not None else None) == 0
        assert np.array_equal(out.view(np.uint32), ro.view(np.uint32))
        if mat is not None:
            R = mat.reshape(dim, dim).astype(np.float64)
            assert np.allclose(R @ R.T, np.eye(dim), atol=1e-6)
            assert np.allclose(x.astype(np.float64) @ R, out, atol=1e-5)
    p = 1 << (dim.bit_length() - 1)
    y = np.empty(dim, np.float32)
    O.or_rot(ptr(out), ptr(y), dim)  # H is symmetric and orthogonal: self-inverse
    assert np.allclose(y[:p], x[:p], atol=1e-5)
    assert np.array_equal(out[p:], x[p:])


# ---- dequant (canonical codebook equivalence) --------------------------------------------

@needs_ref
@pytest.mark.parametrize("bits", [2, 4])
def test_dequant_equals_reference_codebook(O, bits):
    rng = np.random.default_rng(5)
    N, K, G = 32, 256, 128
    C_ = (1 << bits) - 1
    vals = rng.integers(0, C_ + 1, size=(N, K), dtype=np.uint8)
    e = rng.integers(-8, -2, size=K // G)
    s_ref = (C_ / 2.0) * np.exp2(e)                      # exact in fp16
    s_ours = np.exp2(e)                                  # 2 * s_ref / C
    # reference: group-major codes, one scale per group shared by all rows
    gm = np.concatenate([vals[:, g * G:(g + 1) * G].reshape(-1) for g in range(K // G)])
    gm_packed = ia.pack_codes(gm, bits)
    ref_out = np.empty(N * K, np.float32)
    po.ref().ref_dequant(bits, N, K, G, ptr(gm_packed), gm_packed.size,
                    ptr(s_ref.astype(np.float16).view(np.uint16).copy()), K // G, ptr(ref_out))
    lin = ia.HostLinear(N, K, bits, ia.pack_codes(vals, bits),
                        np.tile(s_ours.astype(np.float16).view(np.uint16), (N, 1)).copy(),
                        np.full((N, K // G), C_ / 2.0, np.float16).view(np.uint16).copy(), vals)
    ours = np.empty((N, K), np.float32)
    O.or_dequant(C.byref(lin.struct), ptr(ours))
    assert np.allclose(ours.reshape(-1), ref_out, rtol=2 ** -21, atol=0)
    cb = np.empty(C_ + 1, np.float32)
    po.ref().ref_canonical_codebook(bits, ptr(cb))
    assert np.allclose(cb, (2 * np.arange(C_ + 1) - C_) / C_, atol=1e-7)


# ---- rmsnorm -------------------------------------------------------------------------------

@pytest.mark.parametrize("dim", [128, 1024])
def test_rmsnorm_formula(O, dim):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, size=dim).astype(np.float32)
    w = rng.normal(0, 0.1, size=dim).astype(np.float32)
    out = np.empty(dim, np.float32)
    O.or_rmsnorm(ptr(x), ptr(w), ptr(out), dim, np.float32(1e-6))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean() + 1e-6) * (1 + w.astype(np.float64))
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-6)


# ---- quant GEMM -------------------------------------------------------------------------------

@pytest.mark.parametrize("bits,N,K", [(2, 64, 1024), (4, 48, 2048), (8, 32, 384)])
def test_qgemm_ts_brute_force(bits, N, K):
    rng = np.random.default_rng(7)
    lin = ia.make_linear(N, K, bits, rng)
    a = rng.integers(-127, 128, size=(5, K), dtype=np.int8)
    T, S = po.qgemm_ts(a, lin)
    ng = K // 128
    Te = np.einsum("mgk,ngk->mng", a.astype(np.int64).reshape(5, ng, 128),
                   lin.values.astype(np.int64).reshape(N, ng, 128))
    assert np.array_equal(T, Te.astype(np.int32))
    assert np.array_equal(S, a.astype(np.int64).reshape(5, ng, 128).sum(-1))


@pytest.mark.parametrize("bits", [2, 4])
def test_qgemm_fold_matches_float64_dequant(bits):
    rng = np.random.default_rng(8)
    N, K, M = 96, 1024, 7
    zero = rng.uniform(0, (1 << bits) - 1, size=(N, K // 128))  # general zeros too
    lin = ia.make_linear(N, K, bits, rng, zero=zero)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    q, s, _ = po.act_quant(x)
    out = po.qgemm(q, s[:, 0], lin).view(np.float16).astype(np.float64)
    sc = lin.scale.view(np.float16).astype(np.float64)
    ze = lin.zero.view(np.float16).astype(np.float64)
    W = sc.repeat(128, 1) * (lin.values.astype(np.float64) - ze.repeat(128, 1))
    ref = s[:, :1].astype(np.float64) * (q.astype(np.float64) @ W.T)
    assert np.allclose(out, ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max())


# ---- lm_head ----------------------------------------------------------------------------------

def test_lmhead_quant_closed_form(O):
    rng = np.random.default_rng(9)
    V, H = 64, 256
    W = rng.normal(0, 1, size=(V, H)).astype(np.float32)
    W[3] = 0
    q = np.empty((V, H), np.int8)
    s = np.empty(V, np.uint16)
    O.or_lmhead_quant(ptr(W), V, H, ptr(q), ptr(s))
    for r in range(V):
        mx = np.abs(W[r]).max()
        sc = np.float32(mx / np.float32(127.0)) if mx > 0 else np.float32(1.0)
        assert s[r] == np.float16(sc).view(np.uint16)
        inv = np.float32(np.float32(1.0) / sc)
        assert np.array_equal(q[r], np.rint(W[r] * inv).astype(np.int8))


def test_lmhead_logits_and_first_max(O):
    rng = np.random.default_rng(10)
    V, H, M = 80, 256, 3
    wq = rng.integers(-127, 128, size=(V, H), dtype=np.int8)
    wq[17] = wq[5]  # identical rows -> tied logits, the lower index must win
    ws = np.full(V, 0.01, np.float16).view(np.uint16)
    x = rng.normal(0, 1, size=(M, H)).astype(np.float32)
    x[1] = wq[5].astype(np.float32)  # row 1 prefers vocab 5 (and its tie 17)
    aq, as_, _ = po.act_quant(x, round=1, ga=64)
    logits = np.empty((M, V), np.float32)
    best = np.empty(M, np.int32)
    O.or_lmhead(ptr(aq), ptr(as_), M, ptr(wq), ptr(ws), V, H, ptr(logits), ptr(best))
    ref = (aq.astype(np.float64).reshape(M, H // 64, 64) * as_[:, :, None]).reshape(M, H) @ \
        wq.astype(np.float64).T * float(np.float16(0.01))
    assert np.allclose(logits, ref, rtol=1e-5, atol=1e-4)
    assert best[1] == 5 and logits[1, 5] == logits[1, 17]
    assert all(best[m] == int(np.argmax(logits[m])) for m in range(M))


# ---- attention / rope / kv int8 ------------------------------------------------------------------

def test_attention_row_matches_float64(O):
    rng = np.random.default_rng(11)
    nq, nkv, hd, pos = 16, 8, 128, 77
    q = rng.normal(0, 1, size=nq * hd).astype(np.float32)
    k = rng.normal(0, 1, size=(pos + 1, nkv * hd)).astype(np.float32)
    v = rng.normal(0, 1, size=(pos + 1, nkv * hd)).astype(np.float32)
    out = np.empty(nq * hd, np.float32)
    O.or_attention_row(ptr(q), ptr(k), ptr(v), pos, nq, nkv, hd, ptr(out))
    G = nq // nkv
    qd = q.astype(np.float64).reshape(nq, hd)
    kd = k.astype(np.float64).reshape(pos + 1, nkv, hd)
    vd = v.astype(np.float64).reshape(pos + 1, nkv, hd)
    ref = np.empty((nq, hd))
    for h in range(nq):
        s = kd[:, h // G] @ qd[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h] = p @ vd[:, h // G]
    assert np.allclose(out.reshape(nq, hd), ref, atol=2e-5)


@pytest.mark.parametrize("nq,nkv,pos,split", [(16, 8, 77, 256), (16, 8, 700, 256), (40, 8, 1000, 256),
                                              (16, 8, 1000, 32), (16, 8, 31, 32), (8, 8, 256, 256)])
def test_attention_row_split_order_matches_float64(O, nq, nkv, pos, split):
    """The split-order attention (the device's decomposition: 32-token pages
    with a running base-2 max inside each KV split, splits merged in order)
    is the same softmax attention as float64 -- across page and split
    boundaries, at a split and a page exactly full -- and differs from the
    reference loop order only in the last ulps.  Keys drawn with a growing
    trend make later pages move the running max, so a dropped rescale of the
    sum or of O, or a split weight taken from the wrong max, fails here."""
    rng = np.random.default_rng(pos + split)
    hd, G = 128, nq // nkv
    q = rng.normal(0, 1, size=nq * hd).astype(np.float32)
    k = (rng.normal(0, 1, size=(pos + 1, nkv * hd)) +
         np.linspace(0, 0.3, pos + 1)[:, None] * q.reshape(nq, hd)[::G].reshape(-1)[None, :]).astype(np.float32)
    v = rng.normal(0, 1, size=(pos + 1, nkv * hd)).astype(np.float32)
    out = np.empty(nq * hd, np.float32)
    loop = np.empty(nq * hd, np.float32)
    O.or_attention_row_split(ptr(q), ptr(k), ptr(v), pos, nq, nkv, hd, split, ptr(out))
    O.or_attention_row(ptr(q), ptr(k), ptr(v), pos, nq, nkv, hd, ptr(loop))
    qd = q.astype(np.float64).reshape(nq, hd)
    kd = k.astype(np.float64).reshape(pos + 1, nkv, hd)
    vd = v.astype(np.float64).reshape(pos + 1, nkv, hd)
    ref = np.empty((nq, hd))
    for h in range(nq):
        s = kd[:, h // G] @ qd[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h] = p @ vd[:, h // G]
    assert np.allclose(out.reshape(nq, hd), ref, atol=2e-5)
    assert np.abs(out - loop).max() < 4e-6


def test_rope_matches_float64_of_f32_angle(O):
    rng = np.random.default_rng(12)
    hd, theta = 128, 1e6
    for pos in (0, 1, 17, 999, 8191):
        x = rng.normal(0, 1, size=hd).astype(np.float32)
        y = x.copy()
        O.or_rope(ptr(y), pos, hd, np.float32(theta))
        half = hd // 2
        d = np.arange(half)
        # powf is correctly rounded here: float64 pow rounded once to float32
        pw = np.array([np.float32(float(np.float32(theta)) ** (2.0 * dd / hd)) for dd in d], np.float32)
        inv = (np.float32(1.0) / pw).astype(np.float32)
        f = (inv * np.float32(pos)).astype(np.float32).astype(np.float64)
        a, b = x[:half].astype(np.float64), x[half:].astype(np.float64)
        ref = np.concatenate([a * np.cos(f) - b * np.sin(f), a * np.sin(f) + b * np.cos(f)])
        assert np.allclose(y, ref, atol=3e-6), pos


def test_kv_int8_round_closed_form(O):
    rng = np.random.default_rng(13)
    x = rng.normal(0, 1, size=128).astype(np.float32)
    y = x.copy()
    O.or_kv_int8_round(ptr(y), 128)
    s = np.float32(np.float16(np.abs(x).max() / np.float32(127.0)))
    inv = np.float32(np.float32(1.0) / s)
    t = (x * inv).astype(np.float32)
    q = np.clip(np.trunc(np.where(t >= 0, t + np.float32(0.5), t - np.float32(0.5))), -127, 127)
    assert np.array_equal(y, (q.astype(np.float32) * s).astype(np.float32))


# ---- forward invariants ---------------------------------------------------------------------------

def tiny_cfg(**over):
    return ia.default_cfg(hidden=256, layers=2, n_heads=4, n_kv=2, inter=384, vocab=512, **over)


def test_forward_chunk_invariance():
    """A prefill chunk of 8 rows equals 8 single-row forwards (test_cpu_parity.sh:65-74)."""
    m = ia.SynthModel(tiny_cfg(), seed=21)
    rng = np.random.default_rng(21)
    toks = rng.integers(0, 512, size=12).tolist()
    e1 = po.OracleEngine(m)
    e2 = po.OracleEngine(m)
    s1, s2 = e1.seq_open(), e2.seq_open()
    b1, l1 = e1.forward([(s1, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
    l2 = []
    for p, t in enumerate(toks):
        b, lg = e2.forward([(s2, p, t, 1, 1)], logits=True)
        l2.append(lg[0])
    assert np.array_equal(l1, np.stack(l2))


def test_forward_f32_tracks_a8():
    m = ia.SynthModel(tiny_cfg(), seed=22)
    rng = np.random.default_rng(22)
    toks = rng.integers(0, 512, size=10).tolist()
    outs = []
    for mode in (0, 1):
        e = po.OracleEngine(m, mode=mode)
        s = e.seq_open()
        b, lg = e.forward([(s, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
        outs.append(lg)
    a8, f32 = outs
    for r in range(len(toks)):
        c = np.corrcoef(a8[r], f32[r])[0, 1]
        assert c > 0.98, (r, c)


def test_attn_dispatch_order_invariants():
    """The attention dispatch order restatement: every unit exactly once; the
    4 slots of a chunked workgroup hold the same (kv head, split) of 4
    consecutive q-blocks of one sequence; single-q-block groups are dense."""
    from oracle import pack as pk
    rng = np.random.default_rng(12)
    for trial in range(20):
        rows, seq = [], 0
        for _ in range(int(rng.integers(1, 6))):
            n = int(rng.choice([1, 1, 3, 9, 40, 70]))
            p0 = int(rng.integers(0, 900))
            rows += [(seq, p0 + i, 0, 1, 0) for i in range(n)]
            seq += 1
        nkv, qb, split = 2, 8, 256
        exp = pk.pack(rows, nkv, qb, split)
        order, units = exp["order"], exp["units"]
        assert sorted(u for u in order if u >= 0) == list(range(len(units)))
        for i in range(0, len(order), 4):
            wg = [units[u] for u in order[i:i + 4] if u >= 0]
            if not wg:
                continue
            same = {(u[0], u[1], u[5]) for u in wg}
            if len(wg) > 1 and len(same) == 1:
                q0 = sorted(u[2] for u in wg)
                assert all(b - a == qb for a, b in zip(q0, q0[1:])) or len(q0) == 1
        # the dense tail: single-q-block groups only, in unit order
        single = [u for u, x in enumerate(units) if sum(1 for r in rows if r[0] == x[0]) <= qb]
        tail = [u for u in order[len(order) - len(single):]] if single else []
        assert tail == single


# ---- the forward as a whole, and the attention output gate ---------------------------------------

def _dequant(O, lin):
    w = np.empty(lin.N * lin.K, np.float32)
    O.or_dequant(C.byref(lin), ptr(w))
    return w.reshape(lin.N, lin.K).astype(np.float64)


def _vec(p, n):
    return np.ctypeslib.as_array(p, shape=(n,)).astype(np.float64)


def _np_forward_f32(O, m, toks):
    """float64 restatement of the reference CPU path (step_batch's full-attention
    branch, main.cpp:7519-7772; tied lm_head :8302-8307) for one sequence's
    prompt rows at positions 0..M-1, from the model's own tensors: weights
    dequantized by or_dequant, the rotation as the dense Sylvester Hadamard
    over sqrt(n), RoPE angles in float32 as the oracle forms them, the output
    gate as sigmoid of the gate rows [2h hd + hd, 2h hd + 2 hd) of q_proj."""
    from scipy.linalg import hadamard
    c = m.cfg
    H, hd, nq, nkv, F = c.hidden, c.head_dim, c.n_heads, c.n_kv, c.inter
    G = nq // nkv
    R = hadamard(H).astype(np.float64) / np.sqrt(H)
    rot = (lambda x: x @ R.T) if c.rotate else (lambda x: x)

    def rms(x, w):
        return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + np.float64(np.float32(c.rms_eps))) * (1.0 + w)

    half = c.rotary_dim // 2
    pw = np.array([np.float32(float(np.float32(c.rope_theta)) ** (2.0 * d / c.rotary_dim)) for d in range(half)],
                  np.float32)
    inv = (np.float32(1.0) / pw).astype(np.float32)

    def rope(x, pos):  # x [..., hd]
        f = (inv * np.float32(pos)).astype(np.float32).astype(np.float64)
        a, b = x[..., :half].copy(), x[..., half:2 * half].copy()
        y = x.copy()
        y[..., :half] = a * np.cos(f) - b * np.sin(f)
        y[..., half:2 * half] = a * np.sin(f) + b * np.cos(f)
        return y

    emb = m.embed().astype(np.float64)
    M = len(toks)
    x = emb[toks]
    for l in range(c.layers):
        L = m.layer(l)
        W = {nm: _dequant(O, getattr(L, nm)) for nm in ("q", "k", "v", "o", "gate", "up", "down")}
        r = rot(rms(x, _vec(L.in_ln, H)))
        qo = r @ W["q"].T
        if c.attn_gate:
            qo = qo.reshape(M, nq, 2, hd)
            q, gate = qo[:, :, 0], qo[:, :, 1]
        else:
            q, gate = qo.reshape(M, nq, hd), None
        k = (r @ W["k"].T).reshape(M, nkv, hd)
        v = (r @ W["v"].T).reshape(M, nkv, hd)
        if c.qk_norm:
            q = rms(q, _vec(L.q_norm, hd))
            k = rms(k, _vec(L.k_norm, hd))
        q = np.stack([rope(q[p], p) for p in range(M)])
        k = np.stack([rope(k[p], p) for p in range(M)])
        att = np.zeros((M, nq, hd))
        for p in range(M):
            for h in range(nq):
                s = k[:p + 1, h // G] @ q[p, h] / np.sqrt(hd)
                e = np.exp(s - s.max())
                att[p, h] = (e / e.sum()) @ v[:p + 1, h // G]
        if gate is not None:
            att = att / (1.0 + np.exp(-gate))
        x = x + rot(att.reshape(M, nq * hd) @ W["o"].T)
        r2 = rot(rms(x, _vec(L.post_ln, H)))
        g, u = r2 @ W["gate"].T, r2 @ W["up"].T
        x = x + rot((g / (1.0 + np.exp(-g)) * u) @ W["down"].T)
    return rms(x, _vec(m.model.final_norm, H)) @ emb.T


@pytest.mark.parametrize("gate", [0, 1])
def test_forward_f32_matches_float64_restatement(O, gate):
    """The f32 (reference CpuBackend) forward, composed, against float64:
    a wrong head / gate index, a dropped norm or rotation, a sign in the gate
    or a transposed operand moves the logits far beyond fp32 rounding."""
    m = ia.SynthModel(tiny_cfg(attn_gate=gate), seed=24)
    toks = np.random.default_rng(24).integers(0, 512, size=7).tolist()
    e = po.OracleEngine(m, mode=1)
    s = e.seq_open()
    _, lg = e.forward([(s, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
    ref = _np_forward_f32(O, m, toks)
    for r in range(len(toks)):
        sd = ref[r].std()
        assert np.abs(lg[r] - ref[r]).max() < 1e-4 * sd, (r, np.abs(lg[r] - ref[r]).max() / sd)
    e.close()


def _zero_gate_pair(cfg_kw, seed):
    """A gated model whose gate rows all have scale 0 (gate = 0, sigmoid = 1/2
    exactly) and the ungated model of the same seed with its O projection's
    post factor 1/2: the same forward, bit for bit, in every path (the
    per-token quantization of x / 2 gives the codes of x and half the scale)."""
    gated = ia.SynthModel(tiny_cfg(attn_gate=1, **cfg_kw), seed=seed)
    plain = ia.SynthModel(tiny_cfg(**cfg_kw), seed=seed)
    c = gated.cfg
    hd, nq = c.head_dim, c.n_heads
    for l in range(c.layers):
        q = gated.layer(l).q
        ng = q.K // 128
        sc = np.ctypeslib.as_array(q.scale, shape=(q.N, ng))
        for h in range(nq):
            sc[(2 * h + 1) * hd:(2 * h + 2) * hd] = 0
        plain.ptr.contents.layers[l].o.post = 0.5
    return gated, plain


@pytest.mark.parametrize("mode", [0, 1])
def test_zero_gate_is_half_the_attention_output(mode):
    gated, plain = _zero_gate_pair({}, 25)
    toks = np.random.default_rng(25).integers(0, 512, size=9).tolist()
    out = []
    for m in (gated, plain):
        e = po.OracleEngine(m, mode=mode)
        s = e.seq_open()
        _, lg = e.forward([(s, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
        out.append(lg)
        e.close()
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    # and the gate matters: with its real rows the outputs differ
    e = po.OracleEngine(ia.SynthModel(tiny_cfg(attn_gate=1), seed=25), mode=mode)
    s = e.seq_open()
    _, lg = e.forward([(s, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
    assert not np.array_equal(lg, out[1])


@pytest.mark.parametrize("mode", [0, 1])
def test_gate_off_reads_the_packed_q_and_skips_the_sigmoid(mode):
    """attn_output_gate = false with a packed q_proj (main.cpp:250, :7697):
    the q rows are taken from the [q, gate] layout and the gate is dropped.
    The synthetic gated model's q rows are the ungated model's of the same
    seed (the gate rows come from their own stream), so the forward equals
    the ungated model's bit for bit; with the gate applied it does not."""
    toks = np.random.default_rng(26).integers(0, 512, size=9).tolist()
    out = []
    for kw in ({"attn_gate": 1, "attn_gate_off": 1}, {}, {"attn_gate": 1}):
        e = po.OracleEngine(ia.SynthModel(tiny_cfg(**kw), seed=26), mode=mode)
        s = e.seq_open()
        _, lg = e.forward([(s, p, t, 1, 1) for p, t in enumerate(toks)], logits=True)
        out.append(lg)
        e.close()
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    assert not np.array_equal(out[2], out[1])


# ---- FP16-activation dequant GEMM (the reference's default GPU linear) ----------------------------

def _f32_round(x):
    """The float32 nearest to the exact rational x (ties to even; normal range)."""
    from fractions import Fraction
    if x == 0:
        return np.float32(0.0)
    sgn = -1 if x < 0 else 1
    mag = abs(x)
    e = mag.numerator.bit_length() - mag.denominator.bit_length()
    if Fraction(2) ** e > mag:
        e -= 1
    ulp = Fraction(2) ** (e - 23)
    q = mag / ulp
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return np.float32(sgn * float(fl * ulp))


def _f16_case(O, bits, M, N, K, alpha, seed):
    rng = np.random.default_rng(seed)
    lin = ia.make_linear(N, K, bits, rng)
    a = (rng.standard_normal((M, K)) * 2).astype(np.float16)
    out = np.empty((M, N), np.uint16)
    O.or_qgemm_f16(ptr(a.view(np.uint16)), M, C.byref(lin.struct), np.float32(alpha), ptr(out))
    Cb = (1 << bits) - 1
    if bits == 2:
        cb = np.array([-1.0, np.float32(-1.0) / np.float32(3.0), np.float32(1.0) / np.float32(3.0), 1.0],
                      np.float32)
    else:
        cb = ((np.float32(2) * np.arange(Cb + 1, dtype=np.float32) - np.float32(Cb)) / np.float32(Cb)).astype(np.float32)
    s = lin.scale.view(np.float16).astype(np.float32).reshape(N, K // 128)
    w = (np.repeat(s, 128, axis=1) * np.float32(alpha)).astype(np.float32) * cb[lin.values]
    return a, w.astype(np.float32), out


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_f16_tiled_is_sequential_fp32(O, bits):
    """M > 1: w rounded to fp16, products exact in fp32, one rounded add per k
    in ascending order -- numpy float32, step by step."""
    M, N, K = 3, 48, 256
    a, w, out = _f16_case(O, bits, M, N, K, 0.37, 40 + bits)
    wh = w.astype(np.float16).astype(np.float32)
    acc = np.zeros((M, N), np.float32)
    af = a.astype(np.float32)
    for k in range(K):
        acc = (acc + af[:, k, None] * wh[None, :, k]).astype(np.float32)
    assert np.array_equal(out, acc.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_f16_decode_is_fused_fp32(O, bits):
    """M == 1: w kept in fp32 and acc = fma(a, w, acc) exactly (rational
    arithmetic rounded once per step); the unfused `acc + a * w` differs."""
    from fractions import Fraction
    N, K = 16, 256
    a, w, out = _f16_case(O, bits, 1, N, K, 1.0, 50 + bits)
    af = a.astype(np.float32)
    ref = np.empty(N, np.uint16)
    unfused_differs = False
    for n in range(N):
        acc, acc2 = np.float32(0), np.float32(0)
        for k in range(K):
            acc = _f32_round(Fraction(float(af[0, k])) * Fraction(float(w[n, k])) + Fraction(float(acc)))
            acc2 = np.float32(acc2 + np.float32(af[0, k] * w[n, k]))
        ref[n] = np.float16(acc).view(np.uint16)
        unfused_differs |= acc2 != acc
    assert np.array_equal(out[0], ref)
    assert unfused_differs


def test_qgemm_f16_tracks_float64(O):
    a, w, out = _f16_case(O, 2, 5, 64, 1024, 1.0, 60)
    ref = a.astype(np.float64) @ w.astype(np.float16).astype(np.float64).T
    got = out.view(np.float16).astype(np.float64)
    assert np.allclose(got, ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max())

# ---- W2A8 DPAS fold with grouped activation scales (the reference's act_group) -----------

def _ga_case(O, bits, M, N, K, ga, alpha, seed, a=None, asc=None, lin=None):
    rng = np.random.default_rng(seed)
    lin = lin or ia.make_linear(N, K, bits, rng)
    if a is None:
        a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    if asc is None:
        asc = (rng.random((M, K // ga)) * 0.02 + 1e-3).astype(np.float32)
    out = np.empty((M, N), np.uint16)
    O.or_qgemm_ga(ptr(np.ascontiguousarray(a)), ptr(np.ascontiguousarray(asc, np.float32)), M, ga,
                  C.byref(lin.struct), np.float32(alpha), ptr(out))
    return a, asc, lin, out


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_ga_one_hot_reads_the_right_slice_and_group(O, bits):
    """One nonzero activation at column k: every op but k's has T = S = 0, so
    out = fp16(((as[k / 64] * ws[k / 128]) * alpha) * (2c - C) * (1/C)) with
    slice scales 2^-j and group scales 2^-g (exact products): the output
    names the slice, the group and the code the fold used."""
    N, K, ga, C_ = 16, 512, 64, (1 << bits) - 1
    rng = np.random.default_rng(7)
    lin = ia.make_linear(N, K, bits, rng)
    sc = np.array([2.0 ** -g for g in range(K // 128)], np.float16)
    lin.scale[:] = np.tile(sc.view(np.uint16), (N, 1))
    asc = np.array([[2.0 ** -(j + 1) for j in range(K // ga)]], np.float32)
    for k in (0, 63, 64, 200, 511):
        a = np.zeros((1, K), np.int8)
        a[0, k] = 3
        _, _, _, out = _ga_case(O, bits, 1, N, K, ga, 1.0, 0, a=a, asc=asc, lin=lin)
        c = lin.values[:, k].astype(np.float64)
        x = (2.0 ** -(k // ga + 1)) * (2.0 ** -(k // 128)) * (2 * 3 * c - C_ * 3)
        ref = (x.astype(np.float32) * np.float32(1.0 / C_)).astype(np.float16)
        assert np.array_equal(out[0], ref.view(np.uint16)), (bits, k)


def test_qgemm_ga_unit_scales_round_each_op(O):
    """Unit scales: each op adds x = fl(d * fl(1/3)) (d = 2T - 3S, exact) to
    the fp32 accumulator with one rounding, ops ascending -- exact rational
    arithmetic rounded per step, T and S summed in int64 over each 32-wide
    op."""
    from fractions import Fraction
    M, N, K, ga = 2, 16, 256, 64
    rng = np.random.default_rng(11)
    lin = ia.make_linear(N, K, 2, rng)
    lin.scale[:] = np.float16(1.0).view(np.uint16)
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    asc = np.ones((M, K // ga), np.float32)
    _, _, _, out = _ga_case(O, 2, M, N, K, ga, 1.0, 0, a=a, asc=asc, lin=lin)
    third = Fraction(float(np.float32(1.0) / np.float32(3.0)))
    for m in range(M):
        for n in range(N):
            acc = np.float32(0)
            for o in range(K // 32):
                sl = slice(32 * o, 32 * o + 32)
                T = int(np.dot(a[m, sl].astype(np.int64), lin.values[n, sl].astype(np.int64)))
                S = int(a[m, sl].astype(np.int64).sum())
                x = _f32_round(Fraction(2 * T - 3 * S) * third)
                acc = _f32_round(Fraction(float(acc)) + Fraction(float(x)))
            assert out[m, n] == np.float16(acc).view(np.uint16), (m, n)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_ga_equal_slices_match_per_row_scale(O, bits):
    """GA = K (one scale per row) equals GA = 64 with that scale in every
    slice, bit for bit."""
    M, N, K = 3, 32, 384
    a, asc, lin, out64 = _ga_case(O, bits, M, N, K, 64, 0.73, 20 + bits,
                                  asc=np.repeat(np.float32([[0.011], [0.02], [0.0037]]), 384 // 64, axis=1))
    _, _, _, outK = _ga_case(O, bits, M, N, K, K, 0.73, 0, a=a, asc=np.float32([[0.011], [0.02], [0.0037]]),
                             lin=lin)
    assert np.array_equal(out64, outK)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qgemm_ga_tracks_float64(O, bits):
    """The dequantized product in float64, sum_k as[m][k/64] a(m,k) ws
    alpha (2c - C)/C, within fp16 output rounding."""
    M, N, K, ga = 4, 64, 1024, 64
    a, asc, lin, out = _ga_case(O, bits, M, N, K, ga, 0.5, 30 + bits)
    C_ = (1 << bits) - 1
    s = lin.scale.view(np.float16).astype(np.float64).reshape(N, K // 128)
    w = np.repeat(s, 128, axis=1) * 0.5 * (2.0 * lin.values - C_) / C_
    ar = a.astype(np.float64) * np.repeat(asc.astype(np.float64), ga, axis=1)
    ref = ar @ w.T
    got = out.view(np.float16).astype(np.float64)
    assert np.allclose(got, ref, rtol=2e-3, atol=1e-3 * np.abs(ref).max())
