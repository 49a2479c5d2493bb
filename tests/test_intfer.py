"""The .intfer (INTFER1) reader, writer and host-model mapping (CPU).

Pins, strongest first:
  * the reference's own reader + writer (src/quant/output.cpp:396-603, built
    from its sources into oracle/_ref) reproduce every file the library
    writes byte for byte, and every file crafted here: so the reference
    parser accepts our files and our writer emits the reference writer's
    exact bytes for the same ModelIR;
  * ifr_intfer_dequant equals the reference's dequant_tensor (dashq.cpp:696-707)
    bit for bit on every tensor, and a numpy restatement from the raw bytes
    (group-major, LSB-first, canonical codebook) that needs no reference;
  * the host linears the loader builds (scale = s_g, zero = C/2,
    post = 2*alpha/C) dequantize, through the oracle, to the reference values
    within fp32 rounding;
  * writer -> reader -> host model reproduces the synthetic model exactly;
  * the canonical-Hadamard check rejects the sign-randomized matrix that the
    reference's magnitude-only check accepts (spinquant.cpp:607-629);
  * malformed images are refused with IFR_EINVAL and unsupported content
    with IFR_EDECLINE, and truncated / corrupted images never crash.
Crafted files come from `craft` below: a separate Python writer of the
container, so the reader is not only checked against the library's writer.
"""
import ctypes as C
import json
import struct

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import _abi
from oracle import pyoracle as po

# The pin library is loaded only inside the tests that use it (po.ref()),
# so a run that deselects them (the GPU tests) never maps it.
HAVE_REF = po.REF_LIB.exists()
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built (no reference tree)")

CFG = dict(hidden=256, layers=2, n_heads=2, n_kv=1, head_dim=128, inter=384, vocab=512)
PRE = "model.language_model."
SCHEME = {2: "INT2", 4: "INT4", 8: "INT8", 16: "FP16"}


def small_cfg(**over):
    c = dict(CFG)
    c.update(over)
    return ia.default_cfg(**c)


def arr(p, n, dt):
    return np.ctypeslib.as_array(C.cast(p, C.POINTER(dt)), shape=(n,)).copy()


# ---- an independent writer of the container ---------------------------------------

def pack_lsb(idx: np.ndarray, bits: int) -> bytes:
    idx = idx.astype(np.uint8).reshape(-1)
    if bits == 8:
        return idx.tobytes()
    per = 8 // bits
    idx = np.concatenate([idx, np.zeros((-len(idx)) % per, np.uint8)]).reshape(-1, per)
    out = np.zeros(idx.shape[0], np.uint8)
    for j in range(per):
        out |= idx[:, j] << (j * bits)
    return out.tobytes()


def quant_tensor(name, role, codes, scales_f16, bits, alpha=None, rot_id=0, group=128):
    """A quantized tensor entry: codes [N][K] (values), one fp16 scale per group."""
    N, K = codes.shape
    G = group
    ng = (K + G - 1) // G
    parts = [codes[:, g * G:(g + 1) * G].reshape(-1) for g in range(ng)]
    return dict(name=name, role=role, N=N, K=K, scheme=SCHEME[bits], group=G,
                has_global=alpha is not None, rot_id=rot_id,
                code=pack_lsb(np.concatenate(parts), bits),
                scale=np.asarray(scales_f16, np.float16).tobytes(),
                glob=b"" if alpha is None else struct.pack("<f", alpha))


def f16_tensor(name, role, values):
    v = np.asarray(values, np.float32)
    N, K = (v.shape[0], 1) if v.ndim == 1 else v.shape
    return dict(name=name, role=role, N=N, K=K, scheme="FP16", group=0, has_global=False, rot_id=0,
                code=v.astype(np.float16).tobytes(), scale=b"", glob=b"")


def craft(tensors, rotations=(), model_id="crafted", n_layers=1, *, n_tensors=None, n_rot=None,
          magic=b"INTFER1\0"):
    code = scale = glob = b""
    ents = []
    for t in tensors:
        ents.append(
            '{"name":%s,"role":%s,"N":%d,"K":%d,"qcfg":{"scheme":%s,"group_size":%d,'
            '"scale_dtype":"FP16","has_global_divisor":%s,"act":"FP16","rotation_id":%d},'
            '"code_offset":%d,"code_bytes":%d,"scale_offset":%d,"scale_bytes":%d,'
            '"global_offset":%d,"global_bytes":%d,"est_error":0}' % (
                json.dumps(t["name"]), json.dumps(t["role"]), t["N"], t["K"], json.dumps(t["scheme"]),
                t["group"], "true" if t["has_global"] else "false", t["rot_id"], len(code),
                len(t["code"]), len(scale), len(t["scale"]), len(glob), len(t["glob"])))
        code += t["code"]
        scale += t["scale"]
        glob += t["glob"]
    rents, rot = [], b""
    for rid, site, mat in rotations:
        rents.append('{"id":%d,"site":%s,"dim":%d,"offset":%d}' % (rid, json.dumps(site), mat.shape[0],
                                                                 len(rot)))
        rot += np.asarray(mat, np.float32).tobytes()
    js = ('{"model_id":%s,"n_layers":%d,"version":1,"tensors":[%s],"rotations":[%s]}' % (
        json.dumps(model_id), n_layers, ",".join(ents), ",".join(rents))).encode()
    nt = len(tensors) if n_tensors is None else n_tensors
    nr = len(rotations) if n_rot is None else n_rot
    head = magic + struct.pack("<IIQQQIHQ", 1, nt, len(code), len(scale), len(glob), nr, 0, len(js))
    return head + js + code + scale + glob + rot


def sylvester(n: int) -> np.ndarray:
    i = np.arange(n)
    sign = np.array([[bin(a & b).count("1") & 1 for b in i] for a in i])
    return np.where(sign == 1, -1.0, 1.0).astype(np.float32) * np.float32(1.0 / np.sqrt(np.float32(n)))


def crafted_model(rng, *, q_bits=2, alpha=None, embed_int8=True, lm_head=True, rotations="shared",
                  q_override=None, group=128):
    """A one-layer model in the container (hidden 256, 2 q / 1 kv heads)."""
    H, hd, qN, kvN, F, V = 256, 128, 256, 128, 384, 64
    ts = []
    if embed_int8:
        ts.append(quant_tensor(PRE + "embed_tokens.weight", "EMBED",
                               rng.integers(0, 256, (V, H)), rng.uniform(0.001, 0.01, H // 128), 8))
    else:
        ts.append(f16_tensor(PRE + "embed_tokens.weight", "EMBED", rng.normal(0, 0.02, (V, H))))
    lp = PRE + "layers.0."
    site = {"q": 0, "k": 0, "v": 0, "o": 1, "gate": 2, "up": 2, "down": 3}
    # rotation ids: "shared" 1 + site (spinquant.cpp:505-513); "reordered"
    # arbitrary ids listed in reverse order (lookup is by id); "partial" leaves
    # down_proj unrotated; "signed" uses sign-flipped matrices; "none".
    base = {"shared": 1, "signed": 1, "partial": 1, "reordered": 40, "none": None}[rotations]

    def rid(k):
        if base is None or (rotations == "partial" and k == "down"):
            return 0
        return base + site[k]
    shapes = {"q": (qN, H), "k": (kvN, H), "v": (kvN, H), "o": (H, qN), "gate": (F, H), "up": (F, H),
              "down": (H, F)}
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
             "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    roles = {"q": "ATTN_Q", "k": "ATTN_K", "v": "ATTN_V", "o": "ATTN_O", "gate": "MLP_GATE",
             "up": "MLP_UP", "down": "MLP_DOWN"}
    ts.append(f16_tensor(lp + "input_layernorm.weight", "NORM", rng.normal(0, 0.1, H)))
    ts.append(f16_tensor(lp + "post_attention_layernorm.weight", "NORM", rng.normal(0, 0.1, H)))
    ts.append(f16_tensor(lp + "self_attn.q_norm.weight", "NORM", rng.normal(0, 0.1, hd)))
    ts.append(f16_tensor(lp + "self_attn.k_norm.weight", "NORM", rng.normal(0, 0.1, hd)))
    for k in ("q", "k", "v", "o", "gate", "up", "down"):
        N, K = shapes[k]
        bits = q_bits if k == "q" else (4 if k in ("v", "down") else 2)
        a = alpha if k == "q" else None
        g = group if k == "q" else 128
        if k == "q" and q_override == "fp16":
            ts.append(f16_tensor(lp + names[k] + ".weight", roles[k], rng.normal(0, 0.02, (N, K))))
            continue
        if k == "q" and q_override == "gated":
            N = 2 * N
        ts.append(quant_tensor(lp + names[k] + ".weight", roles[k],
                               rng.integers(0, 1 << bits, (N, K)),
                               rng.uniform(0.005, 0.03, (K + g - 1) // g), bits, alpha=a, rot_id=rid(k),
                               group=g))
    ts.append(f16_tensor(PRE + "norm.weight", "NORM", rng.normal(0, 0.1, H)))
    if lm_head:
        ts.append(f16_tensor("lm_head.weight", "LM_HEAD", rng.normal(0, 0.02, (V, H))))
    rots = []
    if base is not None:
        mat = sylvester(H)
        if rotations == "signed":
            flip = np.where(np.random.default_rng(3).random(H) < 0.5, -1.0, 1.0).astype(np.float32)
            mat = mat * flip[None, :]
        rots = [(base + s, n, mat) for s, n in enumerate(["QKV", "O", "FFN_IN", "FFN_OUT"])]
        if rotations == "reordered":
            rots = rots[::-1]
    return craft(ts, rots, n_layers=1), ts


CRAFT_CFG = dict(hidden=256, layers=1, n_heads=2, n_kv=1, head_dim=128, inter=384, vocab=64)


def numpy_dequant(t: dict) -> np.ndarray:
    """Closed form of the container's dequant from the raw entry bytes."""
    N, K = t["N"], t["K"]
    if t["scheme"] == "FP16":
        return np.frombuffer(t["code"], np.float16).astype(np.float32).reshape(N, K)
    bits = {"INT2": 2, "INT4": 4, "INT8": 8}[t["scheme"]]
    G = t["group"]
    ng = (K + G - 1) // G
    raw = np.frombuffer(t["code"], np.uint8)
    if bits == 8:
        idx = raw.copy()
    else:
        per = 8 // bits
        idx = np.stack([(raw >> (j * bits)) & ((1 << bits) - 1) for j in range(per)], 1).reshape(-1)
    Cm = (1 << bits) - 1
    cb = ((np.float32(2) * np.arange(Cm + 1, dtype=np.float32) - np.float32(Cm)) / np.float32(Cm))
    alpha = np.float32(struct.unpack("<f", t["glob"])[0]) if len(t["glob"]) >= 4 else np.float32(1)
    s = np.frombuffer(t["scale"], np.float16).astype(np.float32) * alpha
    out = np.empty((N, K), np.float32)
    for g in range(ng):
        k0, gl = g * G, min(K, (g + 1) * G) - g * G
        blk = idx[g * N * G: g * N * G + N * gl].reshape(N, gl)
        out[:, k0:k0 + gl] = s[g] * cb[blk]
    return out


# ---- writer -> reader -> host model ----------------------------------------------

@pytest.mark.parametrize("bits,gate", [(2, 0), (4, 0), (8, 0), (0, 0), (2, 1), (0, 1)])
def test_roundtrip_reproduces_synthetic_model(bits, gate):
    cfg = small_cfg(attn_gate=gate)
    m = ia.SynthModel(cfg, 7, bits, intfer_form=True)
    f = ia.IntferFile(m.write_intfer("rt"))
    assert f.counts() == (2 + 2 * 11, 4, 2) and f.model_id() == "rt"
    h = f.host_model(small_cfg())  # the gate is read from the file
    assert h.cfg.rotate == 1 and h.cfg.group_size == 128 and not h.ptr.contents.lm_head
    assert h.cfg.attn_gate == gate and h.cfg.attn_gate_off == 0
    # the caller's attn_output_gate = false survives the load (main.cpp:250)
    assert f.host_model(small_cfg(attn_gate_off=1)).cfg.attn_gate_off == 1
    H, V = cfg.hidden, cfg.vocab
    for l in range(cfg.layers):
        A, B = m.layer(l), h.ptr.contents.layers[l]
        for nm in ("q", "k", "v", "o", "gate", "up", "down"):
            a, b = getattr(A, nm), getattr(B, nm)
            assert (a.N, a.K, a.bits, a.group) == (b.N, b.K, b.bits, b.group)
            nb, ng = a.N * a.K * a.bits // 8, a.N * a.K // 128
            assert np.array_equal(arr(a.codes, nb, C.c_uint8), arr(b.codes, nb, C.c_uint8))
            assert np.array_equal(arr(a.scale, ng, C.c_uint16), arr(b.scale, ng, C.c_uint16))
            assert np.array_equal(arr(a.zero, ng, C.c_uint16), arr(b.zero, ng, C.c_uint16))
            assert a.post == b.post == np.float32(2.0) / np.float32((1 << a.bits) - 1)
        for nm, n in (("in_ln", H), ("post_ln", H), ("q_norm", 128), ("k_norm", 128)):
            assert np.array_equal(arr(getattr(A, nm), n, C.c_float), arr(getattr(B, nm), n, C.c_float))
    assert np.array_equal(arr(m.model.embed, V * H, C.c_float), arr(h.ptr.contents.embed, V * H, C.c_float))
    assert np.array_equal(arr(m.model.final_norm, H, C.c_float), arr(h.ptr.contents.final_norm, H, C.c_float))
    # the same model written again is the same file
    assert h.write_intfer("rt") == m.write_intfer("rt")


def test_unrotated_model_roundtrip():
    cfg = small_cfg(rotate=0)
    m = ia.SynthModel(cfg, 5, 2, intfer_form=True)
    f = ia.IntferFile(m.write_intfer())
    assert f.counts()[1] == 0
    assert all(t["rotation_id"] == 0 for t in f.tensors())
    assert f.host_model(small_cfg(rotate=1)).cfg.rotate == 0  # the file decides


def test_writer_declines_per_row_scales():
    m = ia.SynthModel(small_cfg(), 7, 2)  # default form: per-(row, group) scales
    with pytest.raises(ia.IfrError) as e:
        m.write_intfer()
    assert e.value.code == ia.IFR_EDECLINE


# ---- the reference's own reader / writer / dequant -----------------------------------

@needs_ref
@pytest.mark.parametrize("bits,rotate", [(2, 1), (4, 0), (0, 1)])
def test_reference_reader_reproduces_our_file(bits, rotate):
    m = ia.SynthModel(small_cfg(rotate=rotate), 9, bits, intfer_form=True)
    b = m.write_intfer("intfer-amd")
    assert po.ref_intfer_reserialize(b) == b


@needs_ref
def test_dequant_matches_reference_bit_exact():
    m = ia.SynthModel(small_cfg(), 9, 0, intfer_form=True)
    b = m.write_intfer()
    f = ia.IntferFile(b)
    for i, t in enumerate(f.tensors()):
        ref = po.ref_intfer_dequant(b, t["name"], t["N"], t["K"])
        assert ref is not None
        assert np.array_equal(f.dequant(i).view(np.uint32), ref.view(np.uint32)), t["name"]


@needs_ref
@pytest.mark.parametrize("variant", ["base", "alpha", "int4q", "int8q", "reordered"])
def test_crafted_files_match_reference(variant):
    rng = np.random.default_rng(sum(map(ord, variant)))
    kw = dict(base={}, alpha=dict(alpha=0.37), int4q=dict(q_bits=4), int8q=dict(q_bits=8, alpha=2.5),
              reordered=dict(rotations="reordered"))[variant]
    b, ts = crafted_model(rng, **kw)
    assert po.ref_intfer_reserialize(b) == b  # the crafted image is in the reference's exact format
    f = ia.IntferFile(b)
    for i, t in enumerate(ts):
        ours = f.dequant(i)
        ref = po.ref_intfer_dequant(b, t["name"], t["N"], t["K"])
        assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32)), t["name"]


@needs_ref
def test_sign_randomized_hadamard_is_declined():
    """The reference's magnitude-only check accepts a sign-flipped H and would
    replay it as the plain FWHT; this reader flags it and the loader declines."""
    b, _ = crafted_model(np.random.default_rng(2), rotations="signed")
    f = ia.IntferFile(b)
    assert [po.ref_intfer_rotation_is_hadamard(b, i) for i in range(4)] == [1, 1, 1, 1]
    assert [f.rotation(i)["hadamard"] for i in range(4)] == [0, 0, 0, 0]
    with pytest.raises(ia.IfrError) as e:
        f.host_model(ia.default_cfg(**CRAFT_CFG))
    assert e.value.code == ia.IFR_EDECLINE


# ---- closed forms (no reference needed) ---------------------------------------------

@pytest.mark.parametrize("variant", ["base", "alpha", "int8q"])
def test_dequant_closed_form(variant):
    rng = np.random.default_rng(40 + len(variant))
    kw = dict(base={}, alpha=dict(alpha=0.37), int8q=dict(q_bits=8, alpha=2.5))[variant]
    b, ts = crafted_model(rng, **kw)
    f = ia.IntferFile(b)
    for i, t in enumerate(ts):
        assert np.array_equal(f.dequant(i).view(np.uint32), numpy_dequant(t).view(np.uint32)), t["name"]


def test_rotation_matrices_are_canonical():
    cfg = small_cfg()
    f = ia.IntferFile(ia.SynthModel(cfg, 1, 2, intfer_form=True).write_intfer())
    for i in range(4):
        info, mat = f.rotation(i, with_matrix=True)
        assert info == dict(id=1 + i, site=i, dim=256, hadamard=1)
        assert np.array_equal(mat, sylvester(256))
        hh = mat.astype(np.float64) @ mat.astype(np.float64)
        assert np.allclose(hh, np.eye(256), atol=1e-6)  # symmetric orthogonal: H H = I


@pytest.mark.parametrize("variant", ["base", "alpha", "int8q", "int4q", "gated"])
def test_host_linears_dequantize_to_file_values(variant):
    """scale = s_g, zero = C/2, post = 2*alpha/C reproduces (s_g*alpha)*cb[c];
    a q_proj of 2 * n_heads * head_dim rows (the attention output gate) is
    taken whole and sets attn_gate."""
    rng = np.random.default_rng(77 + len(variant))
    kw = dict(base={}, alpha=dict(alpha=0.37), int8q=dict(q_bits=8, alpha=2.5), int4q=dict(q_bits=4),
              gated=dict(q_override="gated"))[variant]
    b, ts = crafted_model(rng, **kw)
    f = ia.IntferFile(b)
    cfg = ia.default_cfg(**CRAFT_CFG)
    h = f.host_model(cfg)
    L = h.ptr.contents.layers[0]
    for nm, suffix in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                       ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                       ("down", "mlp.down_proj")):
        lin = getattr(L, nm)
        ours = np.empty((lin.N, lin.K), np.float32)
        po.oracle().or_dequant(C.byref(lin), po.ptr(ours))
        ref = f.dequant(f.find(PRE + "layers.0." + suffix + ".weight"))
        assert np.allclose(ours, ref, rtol=3e-7, atol=0), nm
    # host tensors: the INT8 embedding is dequantized, norms and lm_head are fp16 values
    V, H = cfg.vocab, cfg.hidden
    emb = arr(h.ptr.contents.embed, V * H, C.c_float).reshape(V, H)
    assert np.array_equal(emb, f.dequant(f.find(PRE + "embed_tokens.weight")))
    lm = arr(h.ptr.contents.lm_head, V * H, C.c_float).reshape(V, H)
    assert np.array_equal(lm, f.dequant(f.find("lm_head.weight")))
    assert h.cfg.rotate == 1
    assert h.cfg.attn_gate == (variant == "gated")
    assert L.q.N == (2 if variant == "gated" else 1) * cfg.n_heads * cfg.head_dim


def test_forward_of_parsed_model_equals_synthetic(tmp_path):
    """The oracle forward of the parsed host model equals that of the model it
    was written from (the tensors are identical, post != 1 included)."""
    cfg = small_cfg(layers=1)
    m = ia.SynthModel(cfg, 3, 0, intfer_form=True)
    h = ia.IntferFile(m.write_intfer()).host_model(cfg)
    rows = [(0, p, int(t), ia.ROW_PREFILL, int(p == 7)) for p, t in enumerate(range(100, 108))]
    outs = []
    for mod in (m, h):
        o = po.OracleEngine(mod, kv_int8=0, mode=0, max_seqs=2)
        s = o.seq_open()
        best, lg = o.forward([(s, *r[1:]) for r in rows], logits=True)
        outs.append((best, lg))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))


# ---- refusals ----------------------------------------------------------------------

@pytest.mark.parametrize("kw,code", [
    (dict(q_override="fp16"), _abi.IFR_EDECLINE),
    (dict(group=64), _abi.IFR_EDECLINE),
    (dict(rotations="partial"), _abi.IFR_EDECLINE),
])
def test_unsupported_content_declines(kw, code):
    b, _ = crafted_model(np.random.default_rng(5), **kw)
    f = ia.IntferFile(b)
    with pytest.raises(ia.IfrError) as e:
        f.host_model(ia.default_cfg(**CRAFT_CFG))
    assert e.value.code == code


def test_config_mismatch_is_invalid():
    b, _ = crafted_model(np.random.default_rng(6))
    f = ia.IntferFile(b)
    for over in (dict(layers=2), dict(inter=512), dict(vocab=128), dict(n_kv=2)):
        c = dict(CRAFT_CFG)
        c.update(over)
        with pytest.raises(ia.IfrError) as e:
            f.host_model(ia.default_cfg(**c))
        assert e.value.code == ia.IFR_EINVAL, over


def test_missing_tensor_is_invalid():
    rng = np.random.default_rng(8)
    _, ts = crafted_model(rng)
    b = craft([t for t in ts if "k_norm" not in t["name"]])
    with pytest.raises(ia.IfrError) as e:
        ia.IntferFile(b).host_model(ia.default_cfg(**CRAFT_CFG))
    assert e.value.code == ia.IFR_EINVAL and "k_norm" in str(e.value)


def test_malformed_images_are_refused():
    b, ts = crafted_model(np.random.default_rng(9))
    bad = [b[:53], b"INTFER2\0" + b[8:], b[:200], b[:-1],
           craft(ts, n_tensors=len(ts) + 1), craft(ts, n_rot=1)]
    for img in bad:
        with pytest.raises(ia.IfrError) as e:
            ia.IntferFile(img)
        assert e.value.code == ia.IFR_EINVAL
    # a slice that leaves its region
    t0 = dict(ts[0])
    img = craft([t0])
    js_start = 54
    js_len = struct.unpack_from("<Q", img, 46)[0]
    js = img[js_start:js_start + js_len].replace(b'"code_bytes":%d' % len(t0["code"]),
                                                 b'"code_bytes":%d' % (len(t0["code"]) + 1))
    img2 = img[:46] + struct.pack("<Q", len(js)) + js + img[js_start + js_len:]
    with pytest.raises(ia.IfrError) as e:
        ia.IntferFile(img2)
    assert e.value.code == ia.IFR_EINVAL


def test_corrupted_images_never_crash():
    """Truncations and byte flips of a valid image: every outcome is a clean
    status (the parse runs in this process, so a stray access would end it)."""
    b, _ = crafted_model(np.random.default_rng(10), embed_int8=False, lm_head=False)
    rng = np.random.default_rng(11)
    js_len = struct.unpack_from("<Q", b, 46)[0]
    cfg = ia.default_cfg(**CRAFT_CFG)
    outcomes = {}
    for trial in range(400):
        img = bytearray(b)
        if trial % 3 == 0:
            img = img[:int(rng.integers(0, len(b)))]
        else:
            for _ in range(int(rng.integers(1, 4))):
                pos = int(rng.integers(0, 54 + js_len))  # header and JSON: the parsed parts
                img[pos] = int(rng.integers(0, 256))
        try:
            f = ia.IntferFile(bytes(img))
        except ia.IfrError as e:
            outcomes[e.code] = outcomes.get(e.code, 0) + 1
            continue
        try:
            h = f.host_model(cfg)
            h.close()
            outcomes[0] = outcomes.get(0, 0) + 1
        except ia.IfrError as e:
            outcomes[e.code] = outcomes.get(e.code, 0) + 1
        f.close()
    assert set(outcomes) <= {0, ia.IFR_EINVAL, ia.IFR_EDECLINE}
    assert outcomes.get(ia.IFR_EINVAL, 0) > 100
