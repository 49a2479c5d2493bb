"""ctypes bindings of the CPU oracle (test infrastructure only; see __init__)."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libintfer_ref.so"

_o = None
_r = None

P = C.c_void_p
i32, f32, sz = C.c_int32, C.c_float, C.c_size_t


def build(ref: bool = False) -> None:
    """Build liboracle.so (and the reference pin library when ref=True)."""
    targets = ["all"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


def oracle() -> C.CDLL:
    global _o
    if _o is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        protos = {
            "or_f2h": (C.c_uint16, [f32]),
            "or_h2f": (f32, [C.c_uint16]),
            "or_f2h_batch": (None, [P, P, sz]),
            "or_h2f_batch": (None, [P, P, sz]),
            "or_rot": (None, [P, P, C.c_int]),
            "or_fwht": (None, [P, C.c_int]),
            "or_rmsnorm": (None, [P, P, P, C.c_int, f32]),
            "or_act_quant": (None, [P, C.c_int, C.c_int, P, f32, C.c_int, C.c_int, C.c_int, P, P, P]),
            "or_qgemm_ts": (None, [P, C.c_int, P, P, P]),
            "or_qgemm": (None, [P, P, C.c_int, P, P]),
            "or_qgemm_f16": (None, [P, C.c_int, P, f32, P]),
            "or_qgemm_ga": (None, [P, P, C.c_int, C.c_int, P, f32, P]),
            "or_swiglu": (None, [P, P, P, sz]),
            "or_dequant": (None, [P, P]),
            "or_gemm_f32": (None, [P, P, P, C.c_int, C.c_int, C.c_int]),
            "or_lmhead_quant": (None, [P, C.c_int, C.c_int, P, P]),
            "or_lmhead": (None, [P, P, C.c_int, P, P, C.c_int, C.c_int, P, P]),
            "or_argmax": (C.c_int, [P, C.c_int]),
            "or_rope": (None, [P, C.c_int, C.c_int, f32]),
            "or_attention_row": (None, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
            "or_kv_int8_round": (None, [P, C.c_int]),
            "or_kv_int8_round_rows": (None, [P, C.c_long, C.c_int]),
            "or_attention_row_split": (None, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]),
            "or_engine_set_attn_split": (C.c_int, [P, C.c_int]),
            "or_engine_create": (P, [P, C.c_int, C.c_int, C.c_int]),
            "or_engine_destroy": (None, [P]),
            "or_seq_open": (C.c_int, [P]),
            "or_seq_close": (None, [P, C.c_int]),
            "or_seq_truncate": (C.c_int, [P, C.c_int, C.c_int]),
            "or_seq_set_kv": (C.c_int, [P, C.c_int, C.c_int, P, P]),
            "or_forward": (C.c_int, [P, P, C.c_int, P, P]),
            "or_rng_create": (P, [C.c_uint32]),
            "or_rng_free": (None, [P]),
            "or_rng_next": (C.c_uint32, [P]),
            "or_rng_uniform": (f32, [P]),
            "or_sample": (C.c_int, [P, C.c_int, C.c_int, f32, f32, P]),
        }
        for n, (res, args) in protos.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = res, args
        _o = L
    return _o


def ref() -> C.CDLL | None:
    """Reference quant-core pin library, or None where it is not built."""
    global _r
    if _r is None:
        if not REF_LIB.exists():
            return None
        L = C.CDLL(str(REF_LIB))
        protos = {
            "ref_float_to_half": (C.c_uint16, [f32]),
            "ref_half_to_float": (f32, [C.c_uint16]),
            "ref_act_quant_ga64": (None, [P, P, P, sz, C.c_int]),
            "ref_act_quant_scale_inv": (None, [P, sz, sz, P]),
            "ref_avx2_available": (C.c_int, []),
            "ref_rotation_fwht": (C.c_int, [C.c_uint32, P, P, P]),
            "ref_canonical_codebook": (None, [C.c_int, P]),
            "ref_dequant": (None, [C.c_int, C.c_uint32, C.c_uint32, C.c_uint16, P, sz, P,
                                   C.c_uint32, P]),
            "ref_intfer_reserialize": (C.c_int, [P, sz, C.POINTER(P), C.POINTER(sz)]),
            "ref_intfer_dequant": (C.c_long, [P, sz, C.c_char_p, P, sz]),
            "ref_intfer_rotation_is_hadamard": (C.c_int, [P, sz, C.c_int]),
            "ref_free": (None, [P]),
        }
        for n, (res, args) in protos.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = res, args
        _r = L
    return _r


def ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


# ---- the reference's own INTFER1 reader / writer / dequant (needs _ref) ----------

def ref_intfer_reserialize(blob: bytes) -> bytes | None:
    """The image read by the reference reader and written back by the
    reference writer; None if the reader rejects it."""
    out, n = C.c_void_p(), C.c_size_t()
    if ref().ref_intfer_reserialize(blob, len(blob), C.byref(out), C.byref(n)) != 0:
        return None
    try:
        return C.string_at(out, n.value)
    finally:
        ref().ref_free(out)


def ref_intfer_dequant(blob: bytes, name: str, N: int, K: int) -> np.ndarray | None:
    out = np.empty((N, K), np.float32)
    got = ref().ref_intfer_dequant(blob, len(blob), name.encode(), ptr(out), out.size)
    return out if got == N * K else None


def ref_intfer_rotation_is_hadamard(blob: bytes, i: int) -> int:
    return ref().ref_intfer_rotation_is_hadamard(blob, len(blob), i)


# ---- numpy-level helpers --------------------------------------------------------

def act_quant(x: np.ndarray, *, norm_w=None, eps=1e-6, rotate=0, round=0, ga=0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    ns = K // ga if ga else 1
    q = np.empty((M, K), np.int8)
    s = np.empty((M, ns), np.float32)
    g = np.empty((M, K // 128), np.float32)
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    oracle().or_act_quant(ptr(x), M, K, None if nw is None else ptr(nw), eps, rotate, round, ga,
                          ptr(q), ptr(s), ptr(g))
    return q, s, g


def qgemm(a: np.ndarray, ascale: np.ndarray, lin) -> np.ndarray:
    """fp16 bits [M][N] of the GEMM contract.  lin: intfer_amd.HostLinear."""
    M = a.shape[0]
    out = np.empty((M, lin.N), np.uint16)
    s = lin.struct
    oracle().or_qgemm(ptr(np.ascontiguousarray(a)), ptr(np.ascontiguousarray(ascale, np.float32)), M,
                      C.byref(s), ptr(out))
    return out


def qgemm_ts(a: np.ndarray, lin):
    M = a.shape[0]
    ng = lin.K // 128
    T = np.empty((M, lin.N, ng), np.int32)
    S = np.empty((M, ng), np.int32)
    s = lin.struct
    oracle().or_qgemm_ts(ptr(np.ascontiguousarray(a)), M, C.byref(s), ptr(T), ptr(S))
    return T, S


class OracleEngine:
    """The oracle forward (mode 0 = device contract a8, 1 = reference f32 path)."""

    def __init__(self, model, kv_int8=0, mode=0, max_seqs=8, attn_split=0):
        """attn_split > 0: attention in the split order (or_attention_row_split)
        instead of the reference loop order."""
        self.cfg = model.cfg
        self.model = model
        self.h = oracle().or_engine_create(model.ptr, kv_int8, mode, max_seqs)
        if not self.h:
            raise RuntimeError("or_engine_create failed")
        if attn_split:
            assert oracle().or_engine_set_attn_split(self.h, attn_split) == 0

    def seq_open(self) -> int:
        return oracle().or_seq_open(self.h)

    def seq_close(self, s):
        oracle().or_seq_close(self.h, s)

    def seq_truncate(self, s, n):
        return oracle().or_seq_truncate(self.h, s, n)

    def set_kv(self, s, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert oracle().or_seq_set_kv(self.h, s, k.shape[1], ptr(k), ptr(v)) == 0

    def forward(self, rows, logits=False):
        from intfer_amd import rows_array
        arr = rows_array(rows) if not isinstance(rows, C.Array) else rows
        M = len(arr)
        best = np.full(M, -1, np.int32)
        nwant = sum(1 for r in arr if r.want)
        lg = np.empty((nwant, self.cfg.vocab), np.float32) if logits else None
        rc = oracle().or_forward(self.h, C.cast(arr, C.c_void_p), M, ptr(best),
                                 ptr(lg) if logits else None)
        if rc != 0:
            raise RuntimeError(f"or_forward rc={rc}")
        return (best, lg) if logits else best

    def close(self):
        if self.h:
            oracle().or_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
