"""intfer_amd: MI355X-native mixed-batch M-row forward (continuous batching).

Python is only the test/bench harness over the C-ABI in include/intfer_amd.h;
the product is the gfx950 library intfer_amd/libintfer_amd.so (HIP kernels,
the C++ engine and the C++ scheduler).  Names follow the reference engine:
rows, sequences, pages, chunks, drafts.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Iterable, Sequence

import numpy as np

from . import _abi
from ._abi import (KVCfg, Linear, ModelCfg, Row, SchedBackend, SchedCfg, ROW_DECODE, ROW_PREFILL,
                   ROW_VERIFY, LIN_Q, LIN_K, LIN_V, LIN_O, LIN_GATE, LIN_UP, LIN_DOWN, IFR_OK, IFR_EDECLINE, IFR_EINVAL, IFR_ENOMEM, IFR_EDEVICE, IFR_ESTATE,
                   IfrError, check, lib)

__all__ = ["Device", "Engine", "Scheduler", "Rng", "sample", "SynthModel", "HostModelHandle", "IntferFile", "default_cfg", "make_linear", "rows_array",
           "atile", "untile",
           "ROW_DECODE", "ROW_PREFILL", "ROW_VERIFY", "IfrError", "ModelCfg", "KVCfg", "SchedCfg",
           "Row", "Linear", "lib"]


def default_cfg(**over) -> ModelCfg:
    c = ModelCfg()
    lib().ifr_default_cfg(C.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


class HostModelHandle:
    """A host model owned by the library (synthetic or parsed from an
    .intfer file); released with ifr_host_model_free."""

    cfg: ModelCfg
    ptr = None

    @property
    def model(self):
        return self.ptr.contents

    def layer(self, l: int):
        return self.ptr.contents.layers[l]

    def embed(self) -> np.ndarray:
        c = self.cfg
        return np.ctypeslib.as_array(self.ptr.contents.embed, shape=(c.vocab, c.hidden))

    def close(self):
        if self.ptr:
            lib().ifr_host_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def write_intfer(self, model_id: str = "intfer-amd-synthetic") -> bytes:
        """Serialize to the INTFER1 container (ifr_intfer_write)."""
        buf, n = C.c_void_p(), C.c_size_t()
        check(lib().ifr_intfer_write(self.ptr, model_id.encode(), C.byref(buf), C.byref(n)),
              "ifr_intfer_write")
        try:
            return C.string_at(buf, n.value)
        finally:
            lib().ifr_intfer_buffer_free(buf)


class SynthModel(HostModelHandle):
    """Seeded synthetic decoder (owned by the library).  intfer_form draws
    it in the form an .intfer file stores exactly (IFR_SYNTH_INTFER)."""

    def __init__(self, cfg: ModelCfg, seed: int, bits: int = 2, intfer_form: bool = False):
        self.cfg = cfg
        mode = bits | (_abi.IFR_SYNTH_INTFER if intfer_form else 0)
        self.ptr = lib().ifr_synth_model(C.byref(cfg), C.c_uint64(seed), mode)
        if not self.ptr:
            raise ValueError("ifr_synth_model rejected the configuration")


class IntferFile:
    """A parsed .intfer (INTFER1) image; keeps the bytes alive while open."""

    def __init__(self, blob: bytes):
        self._blob = C.create_string_buffer(bytes(blob), len(blob))
        self.ptr = C.c_void_p()
        check(lib().ifr_intfer_open(self._blob, len(blob), C.byref(self.ptr)), "ifr_intfer_open")

    def counts(self):
        nt, nr, nl = C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().ifr_intfer_counts(self.ptr, C.byref(nt), C.byref(nr), C.byref(nl)),
              "ifr_intfer_counts")
        return nt.value, nr.value, nl.value

    def model_id(self) -> str:
        buf = C.create_string_buffer(512)
        check(lib().ifr_intfer_model_id(self.ptr, buf, 512), "ifr_intfer_model_id")
        return buf.value.decode()

    def tensor(self, i: int) -> dict:
        t = _abi.IntferTensor()
        check(lib().ifr_intfer_tensor_info(self.ptr, i, C.byref(t)), "ifr_intfer_tensor_info")
        d = {f: getattr(t, f) for f, _ in t._fields_}
        d["name"] = t.name.decode()
        return d

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.counts()[0])]

    def find(self, name: str) -> int:
        i = C.c_int32()
        check(lib().ifr_intfer_find(self.ptr, name.encode(), C.byref(i)), "ifr_intfer_find")
        return i.value

    def rotation(self, i: int, with_matrix: bool = False):
        r = _abi.IntferRotation()
        mat = None
        if with_matrix:
            r0 = _abi.IntferRotation()
            check(lib().ifr_intfer_rotation_info(self.ptr, i, C.byref(r0), None), "ifr_intfer_rotation_info")
            mat = np.empty((r0.dim, r0.dim), np.float32)
        check(lib().ifr_intfer_rotation_info(self.ptr, i, C.byref(r),
                                             mat.ctypes.data_as(_abi.pf32) if mat is not None else None),
              "ifr_intfer_rotation_info")
        d = {f: getattr(r, f) for f, _ in r._fields_}
        return (d, mat) if with_matrix else d

    def dequant(self, i: int) -> np.ndarray:
        t = self.tensor(i)
        out = np.empty((t["N"], t["K"]), np.float32)
        check(lib().ifr_intfer_dequant(self.ptr, i, out.ctypes.data_as(_abi.pf32)), "ifr_intfer_dequant")
        return out

    def host_model(self, cfg: ModelCfg) -> HostModelHandle:
        h = HostModelHandle()
        ptr = C.POINTER(_abi.HostModel)()
        check(lib().ifr_intfer_host_model(self.ptr, C.byref(cfg), C.byref(ptr)), "ifr_intfer_host_model")
        h.ptr = ptr
        h.cfg = ModelCfg.from_buffer_copy(ptr.contents.cfg)
        return h

    def close(self):
        if self.ptr:
            lib().ifr_intfer_close(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class HostLinear:
    """A logical quantized linear held in numpy arrays (keeps them alive)."""
    N: int
    K: int
    bits: int
    codes: np.ndarray   # packed uint8
    scale: np.ndarray   # uint16 fp16 bits [N][K/128]
    zero: np.ndarray    # uint16 fp16 bits [N][K/128]
    values: np.ndarray  # unpacked uint8 [N][K]
    post: float = 0.0   # output factor (0 reads as 1)

    @property
    def struct(self) -> Linear:
        s = Linear()
        s.N, s.K, s.bits, s.group = self.N, self.K, self.bits, 128
        s.post = self.post
        s.codes = self.codes.ctypes.data_as(C.POINTER(C.c_uint8))
        s.scale = self.scale.ctypes.data_as(C.POINTER(C.c_uint16))
        s.zero = self.zero.ctypes.data_as(C.POINTER(C.c_uint16))
        return s


def pack_codes(vals: np.ndarray, bits: int) -> np.ndarray:
    """Row-major LSB-first packing (reference dashq pack_codes applied row-major)."""
    flat = vals.reshape(-1).astype(np.uint8)
    if bits == 8:
        return flat.copy()
    per = 8 // bits
    flat = flat.reshape(-1, per)
    out = np.zeros(flat.shape[0], dtype=np.uint8)
    for j in range(per):
        out |= (flat[:, j] & ((1 << bits) - 1)) << (j * bits)
    return out


def make_linear(N: int, K: int, bits: int, rng: np.random.Generator, scale_sigma=0.02,
                zero=None, post: float = 0.0) -> HostLinear:
    vals = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    ng = K // 128
    sc = np.abs(rng.normal(0.0, scale_sigma, size=(N, ng))).astype(np.float16).view(np.uint16)
    z = ((1 << bits) - 1) / 2.0 if zero is None else zero
    if np.isscalar(z):
        zz = np.full((N, ng), z, dtype=np.float16).view(np.uint16)
    else:
        zz = np.asarray(z, dtype=np.float16).reshape(N, ng).view(np.uint16)
    return HostLinear(N, K, bits, pack_codes(vals, bits), sc.copy(), zz.copy(), vals, post)


def atile(q: np.ndarray) -> np.ndarray:
    """Row-major int8 [M][K] -> the A-tile byte layout the GEMM entry points
    read (IFR_ATILE_OFF in intfer_amd.h), padded to a multiple of 16 rows."""
    M, K = q.shape
    Mp = (M + 15) // 16 * 16
    p = np.zeros((Mp, K), dtype=np.int8)
    p[:M] = q
    # [mb][m16][kb][kc][k16] -> [mb][kb][kc][m16][k16]
    t = p.reshape(Mp // 16, 16, K // 64, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(t).reshape(-1)


def untile(buf: np.ndarray, M: int, K: int) -> np.ndarray:
    """Inverse of atile: the first M rows as a row-major int8 [M][K]."""
    Mp = (M + 15) // 16 * 16
    t = np.asarray(buf, dtype=np.int8)[:Mp * K].reshape(Mp // 16, K // 64, 4, 16, 16)
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(Mp, K)[:M]


def rows_array(rows: Iterable[Sequence[int]]):
    rows = list(rows)
    arr = (Row * len(rows))()
    for i, r in enumerate(rows):
        seq, pos, tok, kind, want = r
        arr[i].seq, arr[i].pos, arr[i].token, arr[i].kind, arr[i].want = seq, pos, tok, kind, want
    return arr


class DevBuf:
    def __init__(self, dev: "Device", nbytes: int):
        self.dev = dev
        self.nbytes = nbytes
        self.ptr = C.c_void_p()
        check(lib().ifr_malloc(dev.ctx, nbytes, C.byref(self.ptr)), "ifr_malloc")

    @property
    def p(self):
        return self.ptr

    def free(self):
        if self.ptr:
            lib().ifr_free(self.dev.ctx, self.ptr)
            self.ptr = C.c_void_p()


class Device:
    """One HIP context (one stream) on one GPU."""

    def __init__(self, device: int = 0):
        self.ctx = C.c_void_p()
        check(lib().ifr_ctx_create(device, C.byref(self.ctx)), "ifr_ctx_create")
        self._bufs: list[DevBuf] = []

    def alloc(self, nbytes: int) -> DevBuf:
        b = DevBuf(self, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> DevBuf:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        check(lib().ifr_h2d(self.ctx, b.p, arr.ctypes.data_as(C.c_void_p), arr.nbytes), "ifr_h2d")
        return b

    def download(self, b: DevBuf, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(lib().ifr_d2h(self.ctx, out.ctypes.data_as(C.c_void_p), b.p, out.nbytes), "ifr_d2h")
        return out

    def zeros(self, nbytes: int) -> DevBuf:
        b = self.alloc(nbytes)
        check(lib().ifr_memset(self.ctx, b.p, 0, nbytes), "ifr_memset")
        return b

    def sync(self):
        check(lib().ifr_sync(self.ctx), "ifr_sync")

    def stream(self) -> int:
        """The context's HIP stream handle."""
        return lib().ifr_ctx_stream(self.ctx)

    def timer_begin(self):
        check(lib().ifr_timer_begin(self.ctx), "ifr_timer_begin")

    def timer_end(self) -> float:
        """Device milliseconds since timer_begin (waits for the stream)."""
        ms = C.c_double()
        check(lib().ifr_timer_end(self.ctx, C.byref(ms)), "ifr_timer_end")
        return ms.value

    def close(self):
        if self.ctx:
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            lib().ifr_ctx_destroy(self.ctx)
            self.ctx = C.c_void_p()


class Engine:
    """The device forward over one loaded model."""

    def __init__(self, dev: Device, model: HostModelHandle, max_seqs=8, max_seq_tokens=4096,
                 pool_tokens=None, kv_int8=0, max_rows=640, attn_split=0, lanes=0, intfer=None, separate_qk=0,
                 dense_attention=0):
        """Load `model` (a host model), or with intfer= an .intfer file path
        or image for the architecture `model` (a ModelCfg)."""
        self.dev = dev
        self.cfg = model if isinstance(model, ModelCfg) else model.cfg
        kv = KVCfg()
        kv.max_seqs, kv.max_seq_tokens = max_seqs, max_seq_tokens
        kv.pool_tokens = pool_tokens or max_seqs * max_seq_tokens
        kv.kv_int8, kv.max_rows, kv.attn_split, kv.lanes = kv_int8, max_rows, attn_split, lanes
        kv.separate_qk = separate_qk
        kv.dense_attention = dense_attention
        self.kv = kv
        if intfer is None:
            check(lib().ifr_model_load(dev.ctx, model.ptr, C.byref(kv)), "ifr_model_load")
        elif isinstance(intfer, (bytes, bytearray)):
            buf = C.create_string_buffer(bytes(intfer), len(intfer))
            check(lib().ifr_model_load_intfer(dev.ctx, buf, len(intfer), C.byref(self.cfg), C.byref(kv)),
                  "ifr_model_load_intfer")
        else:
            check(lib().ifr_model_load_intfer_file(dev.ctx, str(intfer).encode(), C.byref(self.cfg),
                                                   C.byref(kv)), "ifr_model_load_intfer_file")

    def seq_open(self) -> int:
        s = C.c_int32()
        check(lib().ifr_seq_open(self.dev.ctx, C.byref(s)), "ifr_seq_open")
        return s.value

    def seq_close(self, s: int):
        check(lib().ifr_seq_close(self.dev.ctx, s), "ifr_seq_close")

    def seq_truncate(self, s: int, n: int):
        check(lib().ifr_seq_truncate(self.dev.ctx, s, n), "ifr_seq_truncate")

    def seq_copy_prefix(self, dst: int, src: int, n: int):
        """Give the empty sequence `dst` the first n positions of `src`'s KV."""
        check(lib().ifr_seq_copy_prefix(self.dev.ctx, dst, src, n), "ifr_seq_copy_prefix")

    def seq_len(self, s: int) -> int:
        n = C.c_int32()
        check(lib().ifr_seq_len(self.dev.ctx, s, C.byref(n)), "ifr_seq_len")
        return n.value

    def load_kv(self, s: int, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        check(lib().ifr_seq_load_kv(self.dev.ctx, s, k.shape[1],
                                     k.ctypes.data_as(_abi.pf32), v.ctypes.data_as(_abi.pf32)),
              "ifr_seq_load_kv")

    def forward(self, rows, logits: bool = False):
        arr = rows if isinstance(rows, C.Array) else rows_array(rows)
        M = len(arr)
        best = np.full(M, -1, dtype=np.int32)
        # logits of the want = 2 rows when there are any, else of every scored row
        n2 = sum(1 for r in arr if r.want == 2)
        nwant = n2 if n2 else sum(1 for r in arr if r.want)
        lg = np.empty((nwant, self.cfg.vocab), dtype=np.float32) if logits else None
        check(lib().ifr_forward(self.dev.ctx, arr, M, best.ctypes.data_as(_abi.pi32),
                                lg.ctypes.data_as(_abi.pf32) if logits else None), "ifr_forward")
        return (best, lg) if logits else best

    def attention(self, layer: int, rows, q_fp16: np.ndarray) -> np.ndarray:
        """Joint ragged attention over resident KV; q_fp16 [M][nq][hd] float16."""
        arr = rows if isinstance(rows, C.Array) else rows_array(rows)
        M = len(arr)
        q = np.ascontiguousarray(q_fp16, dtype=np.float16)
        out = np.empty((M, self.cfg.n_heads * self.cfg.head_dim), np.float32)
        check(lib().ifr_attention(self.dev.ctx, layer, arr, M, q.ctypes.data_as(C.c_void_p),
                                  out.ctypes.data_as(_abi.pf32)), "ifr_attention")
        return out

    # ---- the per-linear seam (LinearBackend, main.cpp:455-566) ----
    def linear_lookup(self, name: str):
        """(layer, IFR_LIN_*) of a reference tensor name."""
        l, w = C.c_int32(), C.c_int32()
        check(lib().ifr_linear_lookup(self.dev.ctx, name.encode(), C.byref(l), C.byref(w)), "ifr_linear_lookup")
        return l.value, w.value

    def linear_shape(self, layer: int, which: int):
        n, k = C.c_int32(), C.c_int32()
        check(lib().ifr_linear_shape(self.dev.ctx, layer, which, C.byref(n), C.byref(k)), "ifr_linear_shape")
        return n.value, k.value

    def linear_rot(self, which: int) -> int:
        s = C.c_int32()
        check(lib().ifr_linear_rot(self.dev.ctx, which, C.byref(s)), "ifr_linear_rot")
        return s.value

    def linear_batch(self, layer: int, which: int, X: np.ndarray) -> np.ndarray:
        """run_linear_batch: fp32 [M][N] = W X over host fp32 rows [M][K]."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        N, K = self.linear_shape(layer, which)
        assert X.ndim == 2 and X.shape[1] == K
        Y = np.empty((X.shape[0], N), np.float32)
        check(lib().ifr_linear_batch(self.dev.ctx, layer, which, X.ctypes.data_as(_abi.pf32),
                                     Y.ctypes.data_as(_abi.pf32), X.shape[0]), "ifr_linear_batch")
        return Y

    def linear_wave_batch(self, items, M: int):
        """run_linear_wave_batch over [(layer, which, X)]; returns the Ys."""
        keep, arr = [], (_abi.LinearItem * max(1, len(items)))()
        for i, (l, w, X) in enumerate(items):
            X = np.ascontiguousarray(X, dtype=np.float32)
            N, _ = self.linear_shape(l, w)
            Y = np.empty((M, N), np.float32)
            keep.append((X, Y))
            arr[i] = _abi.LinearItem(l, w, X.ctypes.data_as(_abi.pf32), Y.ctypes.data_as(_abi.pf32))
        check(lib().ifr_linear_wave_batch(self.dev.ctx, arr, len(items), M), "ifr_linear_wave_batch")
        return [y for _, y in keep]

    def mlp_fused(self, layer: int, rin: np.ndarray) -> np.ndarray:
        """run_mlp_fused: md [M][hidden] = W_down(silu(W_gate rin) * (W_up rin))."""
        rin = np.ascontiguousarray(rin, dtype=np.float32)
        md = np.empty((rin.shape[0], self.cfg.hidden), np.float32)
        check(lib().ifr_mlp_fused(self.dev.ctx, layer, rin.ctypes.data_as(_abi.pf32), md.ctypes.data_as(_abi.pf32),
                                  rin.shape[0]), "ifr_mlp_fused")
        return md

    def set_timing(self, on: bool):
        check(lib().ifr_set_timing(self.dev.ctx, 1 if on else 0), "ifr_set_timing")

    def timing(self, kernel: str):
        """(total ms, launches, algorithmic bytes, flops) since set_timing(True)."""
        ms, n, b, f = C.c_double(), C.c_int64(), C.c_double(), C.c_double()
        check(lib().ifr_get_timing(self.dev.ctx, kernel.encode(), C.byref(ms), C.byref(n),
                                   C.byref(b), C.byref(f)), "ifr_get_timing")
        return ms.value, n.value, b.value, f.value


class Scheduler:
    """The C++ continuous-batching scheduler over an Engine, or over a
    backend table (SchedBackend) for CPU-side checks."""

    def __init__(self, engine: Engine | None = None, chunk_m=128, live_cap=64, split_iter=0,
                 round_robin=1, spec_k=0, backend: SchedBackend | None = None, pack_prefill=0,
                 prefix_cache=0, seed=0, spec_adapt=0):
        cfg = SchedCfg()
        cfg.chunk_m, cfg.live_cap, cfg.split_iter = chunk_m, live_cap, split_iter
        cfg.round_robin, cfg.spec_k, cfg.pack_prefill = round_robin, spec_k, pack_prefill
        cfg.prefix_cache, cfg.seed, cfg.spec_adapt = prefix_cache, seed & 0xFFFFFFFF, spec_adapt
        self.h = C.c_void_p()
        self._keep = backend
        if backend is not None:
            check(lib().ifr_sched_create_backend(C.byref(backend), C.byref(cfg), C.byref(self.h)),
                  "ifr_sched_create_backend")
        else:
            check(lib().ifr_sched_create(engine.dev.ctx, C.byref(cfg), C.byref(self.h)),
                  "ifr_sched_create")

    def submit(self, prompt: Sequence[int], max_new: int, temperature: float = 0.0, top_k: int = 0,
               top_p: float = 0.0, seed: int | None = None) -> int:
        """Queue a request; greedy unless a sampling parameter is set."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        rid = C.c_int64()
        sp = _abi.SampleParams(temperature, top_k, top_p, 0 if seed is None else seed & 0xFFFFFFFF,
                               0 if seed is None else 1)
        check(lib().ifr_sched_submit_sampled(self.h, p.ctypes.data_as(_abi.pi32), len(p), max_new,
                                             C.byref(sp), C.byref(rid)), "ifr_sched_submit_sampled")
        return rid.value

    def step(self) -> int:
        n = C.c_int32()
        check(lib().ifr_sched_step(self.h, C.byref(n)), "ifr_sched_step")
        return n.value

    def result(self, rid: int):
        n, done = C.c_int32(), C.c_int32()
        check(lib().ifr_sched_result(self.h, rid, None, 0, C.byref(n), C.byref(done)),
              "ifr_sched_result")
        out = np.zeros(max(n.value, 1), dtype=np.int32)
        check(lib().ifr_sched_result(self.h, rid, out.ctypes.data_as(_abi.pi32), n.value,
                                     C.byref(n), C.byref(done)), "ifr_sched_result")
        return out[:n.value].tolist(), bool(done.value)

    def last_rows(self):
        n = C.c_int32()
        check(lib().ifr_sched_last_rows(self.h, None, 0, C.byref(n)), "ifr_sched_last_rows")
        arr = (Row * max(n.value, 1))()
        check(lib().ifr_sched_last_rows(self.h, arr, n.value, C.byref(n)), "ifr_sched_last_rows")
        return [(r.seq, r.pos, r.token, r.kind, r.want) for r in arr[:n.value]]

    def info(self):
        """(live, prefill queue, pending, per-sequence KV capacity)."""
        v = [C.c_int32() for _ in range(4)]
        check(lib().ifr_sched_info(self.h, *[C.byref(x) for x in v]), "ifr_sched_info")
        return tuple(x.value for x in v)

    def serve(self, lines, vocab: int = 0, default_max_new: int = 64, temperature: float = 0.0,
              top_k: int = 0, top_p: float = 0.0, seed: int = 0):
        """Run the JSON-lines serve loop (ifr_serve) over pipes on `lines`
        (one request per string); returns (output events as dicts, status)."""
        import json
        import os
        import threading
        rin, win = os.pipe()
        rout, wout = os.pipe()
        cfg = _abi.ServeCfg(default_max_new, vocab, temperature, top_k, top_p, seed & 0xFFFFFFFF)
        res = {}

        def run():
            try:
                res["rc"] = lib().ifr_serve(self.h, rin, wout, C.byref(cfg))
            finally:
                os.close(wout)

        def feed():
            with os.fdopen(win, "wb") as f:
                f.write("".join(ln + "\n" for ln in lines).encode())

        th, tw = threading.Thread(target=run), threading.Thread(target=feed)
        th.start()
        tw.start()
        with os.fdopen(rout, "rb") as f:
            out = f.read()
        th.join()
        tw.join()
        os.close(rin)
        return [json.loads(ln) for ln in out.decode().splitlines() if ln.strip()], res.get("rc", -1)

    def close(self):
        if self.h:
            lib().ifr_sched_destroy(self.h)
            self.h = C.c_void_p()


class Rng:
    """A request's sampler state: the library's std::mt19937 (ifr_rng)."""

    def __init__(self, seed: int):
        self.h = C.c_void_p()
        check(lib().ifr_rng_create(seed & 0xFFFFFFFF, C.byref(self.h)), "ifr_rng_create")

    def uniform(self) -> float:
        u = C.c_float()
        check(lib().ifr_rng_uniform(self.h, C.byref(u)), "ifr_rng_uniform")
        return u.value

    def close(self):
        if self.h:
            lib().ifr_rng_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample(logits: np.ndarray, rng: Rng, temperature: float = 0.0, top_k: int = 0, top_p: float = 0.0) -> int:
    """ifr_sample over one row of logits (the reference's sample())."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    t = C.c_int32()
    check(lib().ifr_sample(lg.ctypes.data_as(_abi.pf32), lg.size, top_k, top_p, temperature, rng.h,
                           C.byref(t)), "ifr_sample")
    return t.value
