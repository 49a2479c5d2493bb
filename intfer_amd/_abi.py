"""ctypes view of include/intfer_amd.h.

Loads the in-tree gfx950 library intfer_amd/libintfer_amd.so.  There is no
fallback: if the library is missing the import of anything that needs it
raises, so no caller can silently run a host path instead of the HIP one.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libintfer_amd.so"
HEADER = HERE.parent / "include" / "intfer_amd.h"

IFR_OK, IFR_EDECLINE, IFR_EINVAL, IFR_ENOMEM, IFR_EDEVICE, IFR_ESTATE = 0, -1, -2, -3, -4, -5
ROW_DECODE, ROW_PREFILL, ROW_VERIFY = 0, 1, 2
LIN_Q, LIN_K, LIN_V, LIN_O, LIN_GATE, LIN_UP, LIN_DOWN = range(7)


class ModelCfg(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("layers", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv", C.c_int32), ("head_dim", C.c_int32), ("inter", C.c_int32),
                ("vocab", C.c_int32), ("rotary_dim", C.c_int32), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float), ("group_size", C.c_int32), ("qk_norm", C.c_int32),
                ("rotate", C.c_int32), ("attn_gate", C.c_int32), ("attn_gate_off", C.c_int32)]


class Linear(C.Structure):
    _fields_ = [("N", C.c_int32), ("K", C.c_int32), ("bits", C.c_int32), ("group", C.c_int32),
                ("codes", C.POINTER(C.c_uint8)), ("scale", C.POINTER(C.c_uint16)),
                ("zero", C.POINTER(C.c_uint16)), ("post", C.c_float)]


class LayerW(C.Structure):
    _fields_ = [(n, Linear) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("in_ln", C.POINTER(C.c_float)), ("post_ln", C.POINTER(C.c_float)),
        ("q_norm", C.POINTER(C.c_float)), ("k_norm", C.POINTER(C.c_float))]


class HostModel(C.Structure):
    _fields_ = [("cfg", ModelCfg), ("embed", C.POINTER(C.c_float)),
                ("final_norm", C.POINTER(C.c_float)), ("layers", C.POINTER(LayerW)),
                ("lm_head", C.POINTER(C.c_float))]


IFR_SYNTH_INTFER = 0x100
SCHEME_FP16, SCHEME_INT8, SCHEME_INT4, SCHEME_INT2 = 0, 1, 2, 3
SITE_QKV, SITE_O, SITE_FFN_IN, SITE_FFN_OUT, SITE_NONE = 0, 1, 2, 3, 4


class IntferTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("role", C.c_int32), ("N", C.c_int32), ("K", C.c_int32),
                ("scheme", C.c_int32), ("group_size", C.c_int32), ("scale_dtype", C.c_int32),
                ("has_global_divisor", C.c_int32), ("act", C.c_int32), ("rotation_id", C.c_int32),
                ("code_offset", C.c_uint64), ("code_bytes", C.c_uint64),
                ("scale_offset", C.c_uint64), ("scale_bytes", C.c_uint64),
                ("global_offset", C.c_uint64), ("global_bytes", C.c_uint64),
                ("est_error", C.c_float)]


class IntferRotation(C.Structure):
    _fields_ = [("id", C.c_int32), ("site", C.c_int32), ("dim", C.c_int32), ("hadamard", C.c_int32)]


class KVCfg(C.Structure):
    _fields_ = [("max_seqs", C.c_int32), ("max_seq_tokens", C.c_int32),
                ("pool_tokens", C.c_int32), ("kv_int8", C.c_int32), ("max_rows", C.c_int32),
                ("attn_split", C.c_int32), ("lanes", C.c_int32), ("separate_qk", C.c_int32),
                ("dense_attention", C.c_int32)]


class Row(C.Structure):
    _fields_ = [("seq", C.c_int32), ("pos", C.c_int32), ("token", C.c_int32),
                ("kind", C.c_int32), ("want", C.c_int32)]


class LinearItem(C.Structure):
    _fields_ = [("layer", C.c_int32), ("which", C.c_int32), ("X", C.POINTER(C.c_float)),
                ("Y", C.POINTER(C.c_float))]


class SchedCfg(C.Structure):
    _fields_ = [("chunk_m", C.c_int32), ("live_cap", C.c_int32), ("split_iter", C.c_int32),
                ("round_robin", C.c_int32), ("spec_k", C.c_int32), ("pack_prefill", C.c_int32),
                ("prefix_cache", C.c_int32), ("seed", C.c_uint32), ("spec_adapt", C.c_int32)]


SEQ_OPEN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_int32))
SEQ_CLOSE = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32)
SEQ_TRUNC = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32, C.c_int32)
FORWARD = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(Row), C.c_int32, C.POINTER(C.c_int32))
SEQ_COPY = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32, C.c_int32, C.c_int32)
FORWARD_LOGITS = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(Row), C.c_int32, C.POINTER(C.c_int32),
                             C.POINTER(C.c_float))


class SampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("seed", C.c_uint32), ("has_seed", C.c_int32)]


class SchedEvent(C.Structure):
    _fields_ = [("id", C.c_int64), ("token", C.c_int32), ("done", C.c_int32), ("generated", C.c_int32),
                ("reserved", C.c_int32)]


class ServeCfg(C.Structure):
    _fields_ = [("default_max_new", C.c_int32), ("vocab", C.c_int32), ("temperature", C.c_float),
                ("top_k", C.c_int32), ("top_p", C.c_float), ("seed", C.c_uint32)]


class SchedBackend(C.Structure):
    _fields_ = [("user", C.c_void_p), ("seq_open", SEQ_OPEN), ("seq_close", SEQ_CLOSE),
                ("seq_truncate", SEQ_TRUNC), ("forward", FORWARD), ("kv_capacity", C.c_int32),
                ("seq_copy_prefix", SEQ_COPY), ("forward_logits", FORWARD_LOGITS), ("vocab", C.c_int32)]


P = C.c_void_p
i32, i64, f32, sz = C.c_int32, C.c_int64, C.c_float, C.c_size_t
pi32, pf32 = C.POINTER(C.c_int32), C.POINTER(C.c_float)

_PROTOS = {
    "ifr_last_error": (C.c_char_p, []),
    "ifr_synth_model": (C.POINTER(HostModel), [C.POINTER(ModelCfg), C.c_uint64, i32]),
    "ifr_synth_free": (None, [C.POINTER(HostModel)]),
    "ifr_host_model_free": (None, [C.POINTER(HostModel)]),
    "ifr_intfer_open": (C.c_int, [P, sz, C.POINTER(P)]),
    "ifr_intfer_close": (C.c_int, [P]),
    "ifr_intfer_counts": (C.c_int, [P, pi32, pi32, pi32]),
    "ifr_intfer_model_id": (C.c_int, [P, C.c_char_p, sz]),
    "ifr_intfer_tensor_info": (C.c_int, [P, i32, C.POINTER(IntferTensor)]),
    "ifr_intfer_find": (C.c_int, [P, C.c_char_p, pi32]),
    "ifr_intfer_rotation_info": (C.c_int, [P, i32, C.POINTER(IntferRotation), pf32]),
    "ifr_intfer_dequant": (C.c_int, [P, i32, pf32]),
    "ifr_intfer_host_model": (C.c_int, [P, C.POINTER(ModelCfg), C.POINTER(C.POINTER(HostModel))]),
    "ifr_intfer_write": (C.c_int, [C.POINTER(HostModel), C.c_char_p, C.POINTER(P), C.POINTER(sz)]),
    "ifr_intfer_buffer_free": (None, [P]),
    "ifr_model_load_intfer": (C.c_int, [P, P, sz, C.POINTER(ModelCfg), C.POINTER(KVCfg)]),
    "ifr_model_load_intfer_file": (C.c_int, [P, C.c_char_p, C.POINTER(ModelCfg), C.POINTER(KVCfg)]),
    "ifr_default_cfg": (None, [C.POINTER(ModelCfg)]),
    "ifr_ctx_create": (C.c_int, [i32, C.POINTER(P)]),
    "ifr_ctx_destroy": (C.c_int, [P]),
    "ifr_sync": (C.c_int, [P]),
    "ifr_malloc": (C.c_int, [P, sz, C.POINTER(P)]),
    "ifr_free": (C.c_int, [P, P]),
    "ifr_h2d": (C.c_int, [P, P, P, sz]),
    "ifr_d2h": (C.c_int, [P, P, P, sz]),
    "ifr_memset": (C.c_int, [P, P, C.c_int, sz]),
    "ifr_linear_upload": (C.c_int, [P, C.POINTER(Linear), C.POINTER(P)]),
    "ifr_linear_upload_pair": (C.c_int, [P, C.POINTER(Linear), C.POINTER(Linear), C.POINTER(P)]),
    "ifr_linear_free": (C.c_int, [P, P]),
    "ifr_linear_bytes": (sz, [P]),
    "ifr_act_quant": (C.c_int, [P, P, i32, i32, P, f32, i32, i32, i32, P, P, P]),
    "ifr_quant_gemm": (C.c_int, [P, P, P, P, P, i32, P, P]),
    "ifr_quant_gemm_swiglu": (C.c_int, [P, P, P, P, P, i32, P]),
    "ifr_quant_gemm_variants": (C.c_int, []),
    "ifr_ctx_stream": (C.c_void_p, [P]),
    "ifr_timer_begin": (C.c_int, [P]),
    "ifr_d2d": (C.c_int, [P, P, P, C.c_size_t]),
    "ifr_timer_end": (C.c_int, [P, C.POINTER(C.c_double)]),
    "ifr_quant_gemm_variant": (C.c_int, [P, P, P, P, P, i32, P, i32]),
    "ifr_quant_gemm_rows": (C.c_int, [P, P, P, P, P, P, i32, P, i32]),
    "ifr_quant_gemm_f16": (C.c_int, [P, P, P, i32, C.c_float, P]),
    "ifr_quant_gemm_ga": (C.c_int, [P, P, P, P, i32, i32, C.c_float, P]),
    "ifr_model_load": (C.c_int, [P, C.POINTER(HostModel), C.POINTER(KVCfg)]),
    "ifr_seq_open": (C.c_int, [P, pi32]),
    "ifr_model_info": (C.c_int, [P, C.POINTER(ModelCfg)]),
    "ifr_sched_submit_sampled": (C.c_int, [P, pi32, i32, i32, C.POINTER(SampleParams), C.POINTER(i64)]),
    "ifr_rng_create": (C.c_int, [C.c_uint32, C.POINTER(P)]),
    "ifr_rng_free": (None, [P]),
    "ifr_rng_uniform": (C.c_int, [P, pf32]),
    "ifr_sample": (C.c_int, [pf32, i32, i32, f32, f32, P, pi32]),
    "ifr_seq_close": (C.c_int, [P, i32]),
    "ifr_seq_truncate": (C.c_int, [P, i32, i32]),
    "ifr_seq_len": (C.c_int, [P, i32, pi32]),
    "ifr_seq_copy_prefix": (C.c_int, [P, i32, i32, i32]),
    "ifr_kv_capacity": (C.c_int, [P, pi32]),
    "ifr_seq_load_kv": (C.c_int, [P, i32, i32, pf32, pf32]),
    "ifr_forward": (C.c_int, [P, C.POINTER(Row), i32, pi32, pf32]),
    "ifr_attention": (C.c_int, [P, i32, C.POINTER(Row), i32, P, pf32]),
    "ifr_attention_noalloc": (C.c_int, [P, i32, C.POINTER(Row), i32, P, P]),
    "ifr_peak_read": (C.c_int, [P, P, sz, i32, C.POINTER(C.c_double)]),
    "ifr_peak_mfma": (C.c_int, [P, i32, i32, i32, C.POINTER(C.c_double)]),
    "ifr_linear_lookup": (C.c_int, [P, C.c_char_p, C.POINTER(i32), C.POINTER(i32)]),
    "ifr_linear_shape": (C.c_int, [P, i32, i32, C.POINTER(i32), C.POINTER(i32)]),
    "ifr_linear_rot": (C.c_int, [P, i32, C.POINTER(i32)]),
    "ifr_linear_batch": (C.c_int, [P, i32, i32, pf32, pf32, i32]),
    "ifr_linear_wave_batch": (C.c_int, [P, C.POINTER(LinearItem), i32, i32]),
    "ifr_mlp_fused": (C.c_int, [P, i32, pf32, pf32, i32]),
    "ifr_set_timing": (C.c_int, [P, i32]),
    "ifr_get_timing": (C.c_int, [P, C.c_char_p, C.POINTER(C.c_double), C.POINTER(i64),
                                 C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "ifr_debug_pack": (C.c_int, [P, i32, P, P, P, P, P, P, pi32, pi32]),
    "ifr_debug_attn_order": (C.c_int, [P, P, i32, pi32]),
    "ifr_debug_last_lanes": (C.c_int, [P, pi32]),
    "ifr_sched_create": (C.c_int, [P, C.POINTER(SchedCfg), C.POINTER(P)]),
    "ifr_sched_create_backend": (C.c_int, [C.POINTER(SchedBackend), C.POINTER(SchedCfg),
                                           C.POINTER(P)]),
    "ifr_sched_destroy": (C.c_int, [P]),
    "ifr_sched_submit": (C.c_int, [P, pi32, i32, i32, C.POINTER(i64)]),
    "ifr_sched_step": (C.c_int, [P, pi32]),
    "ifr_sched_result": (C.c_int, [P, i64, pi32, i32, pi32, pi32]),
    "ifr_sched_last_rows": (C.c_int, [P, C.POINTER(Row), i32, pi32]),
    "ifr_sched_record_events": (C.c_int, [P, i32]),
    "ifr_sched_events": (C.c_int, [P, C.POINTER(SchedEvent), i32, pi32]),
    "ifr_sched_release": (C.c_int, [P, i64]),
    "ifr_sched_info": (C.c_int, [P, pi32, pi32, pi32, pi32]),
    "ifr_serve": (C.c_int, [P, i32, i32, C.POINTER(ServeCfg)]),
}

_lib = None


def header_functions() -> list[str]:
    """Names of every function the public header declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(ifr_[a-z0-9_]+)\s*\(", text)
    return sorted(set(n for n in names if not n.endswith("_fn")))


def lib() -> C.CDLL:
    """The loaded HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; "
                               "g.build()'` (there is no non-HIP fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class IfrError(RuntimeError):
    def __init__(self, code: int, where: str):
        msg = lib().ifr_last_error().decode(errors="replace")
        super().__init__(f"{where} failed ({code}): {msg}")
        self.code = code


def check(code: int, where: str) -> None:
    if code != IFR_OK:
        raise IfrError(code, where)
