#!/usr/bin/env python3
"""Headline benchmark: continuous-batching serve load on the 0.8B-class INT2
engine at concurrency C=64, one MI355X.

A step is one complete C=64 serve load: 64 synthetic requests (uniform
token-id prompts of length U[64, 2048], max_new 64, greedy) are submitted at
once and the C++ scheduler runs joint iterations (decode rows + a 512-row
prefill chunk, round-robin) until every request is done.  value = output
tokens (64 per request) / wall time of the timed steps.  Weights, KV and all
intermediates are resident in HBM before the timed region starts.

Extra objects on the JSON line:
  roofline      dominant kernel of the load, from HIP events on the engine's
                stream (achieved algorithmic GB/s vs 8 TB/s)
  serve_roofline achieved decode tok/s vs the per-iteration roofline
                t_roof(i) = max(HBM bytes / 8 TB/s, GEMM int8 ops / 5 POP/s +
                attention flops / 2.5 PFLOP/s)
  peaks         measured device peaks (a 2 GiB read stream, int8 and fp16
                MFMA loops); every roofline object also carries frac_measured,
                its achieved rate over the measured peak of the same unit
  cpu_baseline  the reference CPU path (oracle f32 mode: CpuBackend FP32
                dequant GEMM, host attention, serial tied lm_head), timed on a
                bounded sample of the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12
INT8_PEAK = 5.0e15
FP16_PEAK = 2.5e15


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--concurrency", type=int, default=64)
    ap.add_argument("--max-new", type=int, default=64)
    ap.add_argument("--chunk", type=int, default=512)
    ap.add_argument("--kv-int8", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--lanes", type=int, default=0,
                    help="concurrent sub-batches per forward (ifr_kv_cfg.lanes; 0: the engine default, 1)")
    ap.add_argument("--attn-split", type=int, default=0,
                    help="KV tokens per attention unit of the load's engine (0: the library default, 256)")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-gemm", action="store_true", help="skip the decode-GEMM secondary measurement")
    ap.add_argument("--no-packed", action="store_true",
                    help="skip the secondary pack_prefill measurement of the same load")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="run only the cache-cold cfg2 GEMM sweep and print its JSON line")
    ap.add_argument("--gemm-mall", action="store_true",
                    help="--gemm-variants with 100 MB of weight copies (MALL-resident, as in the serve load)")
    ap.add_argument("--gemm-ms", default="128,256,576,1024", help="M values of --gemm-variants")
    ap.add_argument("--gemm-variants", action="store_true",
                    help="time every quant-GEMM launch shape on the 0.8B shapes and print a JSON line")
    ap.add_argument("--gemm-decode", action="store_true",
                    help="every launch shape at decode M (1, 8, 16) on the 0.8B projections")
    ap.add_argument("--gemm-decode-27b", action="store_true",
                    help="every launch shape at decode M (1, 8, 16) on the 27B-class projections, then at "
                         "M = 1, 4 with A also row-major (ifr_quant_gemm_rows)")
    ap.add_argument("--gemm-variants-27b", action="store_true",
                    help="the same on the 27B-class (cfg5) shapes at M = 512 and 2160")
    ap.add_argument("--attn-sweep", action="store_true",
                    help="run only the attention sweep (cfg3, C=64 decode, mixed) and print its JSON line")
    ap.add_argument("--attn-case", default="",
                    help="NAME[:KV8[:REPS]]: repeat one attention case of --attn-sweep (for rocprofv3)")
    ap.add_argument("--attn-splits", default="0",
                    help="comma-separated KV tokens per attention unit for --attn-sweep (0: default)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="run only 8 device copies of 1 GiB (HBM traffic counter calibration)")
    ap.add_argument("--peaks", action="store_true",
                    help="measure only the device peaks (1 GiB read stream, int8 and fp16 MFMA loops)")
    ap.add_argument("--cfg5", action="store_true",
                    help="run only the cfg5 27B-class mixed iteration (M ~ 2160) and print its JSON line")
    ap.add_argument("--cpu-full", action="store_true",
                    help="run only the full CPU-baseline plan (cfg1 iteration, cfg2 fp32 GEMMs, cfg4 "
                         "decode windows at C=1 / 4 and the extrapolated loads) and print its JSON line")
    ap.add_argument("--f16-gemm", action="store_true",
                    help="time the FP16-activation dequant GEMM (the reference's default linear) on the 0.8B "
                         "projections at M = 1, 16, 576 and print its JSON line")
    ap.add_argument("--ga-gemm", action="store_true",
                    help="time the grouped-activation DPAS-fold GEMM (64-wide activation slices) on the 0.8B "
                         "projections at M = 1, 16, 576 and print its JSON line")
    ap.add_argument("--gemm-case", default="",
                    help="NAME:M[:REPS] (qkv, o, gate_up, down, c5gu, c5down): repeat one cache-cold "
                         "GEMM launch shape (for counter collection) and print its JSON line")
    return ap.parse_args()


def log(msg):
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def run_load(ia, eng, prompts, max_new, chunk, record=None, pack=0):
    sch = ia.Scheduler(eng, chunk_m=chunk, live_cap=64, pack_prefill=pack)
    ids = [sch.submit(p, max_new) for p in prompts]
    done_at = {}
    iters = rows = 0
    t0 = time.perf_counter()
    while True:
        n = sch.step()
        iters += 1
        rows += n
        if record is not None:
            record.append(sch.last_rows())
        if n == 0:
            fin = [sch.result(i)[1] for i in ids]
            if all(fin):
                break
        if iters % 16 == 0 or n == 0:
            now = time.perf_counter()
            for i in ids:
                if i not in done_at and sch.result(i)[1]:
                    done_at[i] = now - t0
    t1 = time.perf_counter()
    for i in ids:
        done_at.setdefault(i, t1 - t0)
    toks = len(ids) * max_new
    sch.close()
    return t1 - t0, toks, iters, rows, sorted(done_at.values())


def pct(xs, p):
    s = sorted(xs)
    k = (len(s) - 1) * p / 100.0
    f, c = int(k), min(int(k) + 1, len(s) - 1)
    return s[f] + (s[c] - s[f]) * (k - f)


def serve_roofline(cfg, weight_bytes, lm_bytes, iters_rows, kv_elem, bw=None, i8=None, f16=None):
    """Sum of per-iteration roofline times and decode tokens (decode rows);
    the nominal peaks unless measured ones are given."""
    bw, i8, f16 = bw or HBM_PEAK, i8 or INT8_PEAK, f16 or FP16_PEAK
    H, L, nq, nkv, hd = cfg.hidden, cfg.layers, cfg.n_heads, cfg.n_kv, cfg.head_dim
    F, V = cfg.inter, cfg.vocab
    macs_tok = L * (H * (nq * hd + 2 * nkv * hd) + nq * hd * H + H * 2 * F + F * H)
    kv_tok = L * nkv * hd * 2 * kv_elem
    t_roof = 0.0
    dec = 0
    for rows in iters_rows:
        if not rows:
            continue
        M = len(rows)
        want = sum(r[4] for r in rows)
        dec += sum(1 for r in rows if r[3] == 0)
        # KV read per sequence: its length after the iteration
        seq_len = {}
        for r in rows:
            seq_len[r[0]] = max(seq_len.get(r[0], 0), r[1] + 1)
        B = weight_bytes + (lm_bytes if want else 0) + sum(seq_len.values()) * kv_tok
        ops = 2.0 * M * macs_tok + 2.0 * want * V * H
        fl = sum(4.0 * nq * hd * (r[1] + 1) * L for r in rows)
        t_roof += max(B / bw, ops / i8 + fl / f16)
    return t_roof, dec


GEMMS = ["qgemm_qkv", "qgemm_o", "qgemm_gate_up", "qgemm_down"]
KERNELS = GEMMS + ["attention", "row_quant", "qk_rope_kv", "combine", "quant_plain", "lmhead", "pack"]
# the rocprofv3 kernel names each timing category covers (each GEMM category:
# qgemm_splitk<...> for M <= 64, qgemm_rows<...> above)
ROCPROF_NAMES = {"attention": "attn_kernel<{kv}, 1>",
                 "combine": "combine_kernel<8>", "row_quant": "row_quant1024_kernel",
                 "quant_plain": "quant_plain8<384>", "qk_rope_kv": "qk_rope_kv_kernel",
                 "lmhead": "lmhead_kernel<...> + argmax_final_kernel", "pack": "pack_kernel"}
PEAK_FLOPS = {"qgemm": INT8_PEAK, "attention": FP16_PEAK, "lmhead": INT8_PEAK, **{g: INT8_PEAK for g in GEMMS}}


def traffic_from_profile(kernel, kv_int8):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), read from the committed summary."""
    f = ROOT / "profiles" / f"{kernel}_cfg4_c64{'_kv8' if kv_int8 else ''}_pmc.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def rocprof_avg_us(rocprof_kernel):
    """Average duration of one kernel in the committed rocprofv3 kernel-trace
    summary of the same load (profiles/serve_load_cfg4_c64_kernel_stats.md)."""
    f = ROOT / "profiles" / "serve_load_cfg4_c64_kernel_stats.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        cells = [c.strip().strip("`") for c in line.split("|")]
        if len(cells) > 4 and cells[1].replace("void ", "") == rocprof_kernel:
            try:
                return float(cells[4])
            except ValueError:
                return None
    return None


def kernel_roofline(name, st, kv_int8, brief=False):
    """Roofline of one timing category over the load: bound = the resource
    whose peak time (algorithmic bytes / 8 TB/s or work / MFMA peak) is larger."""
    ms, n, b, f = st
    sec = ms * 1e-3
    pk = PEAK_FLOPS.get(name)
    t_hbm = b / HBM_PEAK
    t_cmp = f / pk if pk else 0.0
    if pk and t_cmp > t_hbm:
        ach = f / sec / 1e12 if sec else 0.0
        r = {"bound": "mfma", "achieved": round(ach, 2), "peak": pk / 1e12, "unit": "TFLOP/s",
             "frac": round(ach * 1e12 / pk, 4)}
    else:
        ach = b / sec / 1e9 if sec else 0.0
        r = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
             "frac": round(ach * 1e9 / HBM_PEAK, 4)}
    r.update({"launches": n, "avg_us": round(1e3 * ms / n, 2) if n else None, "total_ms": round(ms, 2)})
    if brief:
        return r
    tr = traffic_from_profile(name, kv_int8)
    r["traffic"] = round(tr) if tr is not None else None
    rk = ROCPROF_NAMES.get(name, name).format(kv="true" if kv_int8 else "false")
    ra = rocprof_avg_us(rk)
    r["basis"] = ("avg_us: HIP events around every launch of this kind on the engine stream in a "
                  "separate timing pass of the same load (the event pairs add gaps between launches); "
                  "rocprof_avg_us: the committed rocprofv3 kernel-trace average of the same kernel")
    r["rocprof_avg_us"] = ra
    if ra and n:
        per = (f if r["bound"] == "mfma" else b) / n
        r["frac_rocprof"] = round(per / (ra * 1e-6) / (pk if r["bound"] == "mfma" else HBM_PEAK), 4)
    r.update({"kernel": name, "rocprof_kernel": rk,
              "bytes_per_launch": round(b / n) if n else None,
              "flops_per_launch": round(f / n) if n else None,
              "peak_time_us": {"hbm": round(t_hbm / n * 1e6, 2) if n else None,
                               "mfma": round(t_cmp / n * 1e6, 2) if n else None}})
    return r


def gemm_sweep(ia, dev, bits_list=(2, 4), Ms=(1, 8, 16, 64, 256, 1024), reps=3):
    """cfg2: the four 0.8B GEMM shapes, cache-cold.  Each timed pass launches
    the GEMM once on each of R distinct weight copies (R * weight bytes >
    320 MB, above the 256 MB MALL), bracketed by HIP events on the engine
    stream; the best of `reps` passes is reported."""
    import ctypes as C
    L = ia.lib()
    shapes = [("qkv", 1024, 4096), ("o", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)]
    rng = np.random.default_rng(0)
    res = []
    Mmax = max(Ms)
    for bits in bits_list:
        for name, K, N in shapes:
            lin = ia.make_linear(N, K, bits, rng)
            wb = N * K * bits // 8 + N * (K // 128) * 4
            R = int(np.ceil(320e6 / wb))
            dls = []
            for _ in range(R):
                d = C.c_void_p()
                ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(d)), "upload")
                dls.append(d)
            q = dev.upload(rng.integers(-127, 128, size=((Mmax + 15) // 16 * 16) * K, dtype=np.int8))
            asc = dev.upload(np.full(Mmax, 1e-3, dtype=np.float32))
            gs = dev.upload(rng.integers(-2000, 2000, size=Mmax * (K // 128)).astype(np.float32))
            out = dev.alloc(Mmax * N * 2)
            for M in Ms:
                best = None
                for _ in range(reps + 1):  # first pass warms code and TLB
                    dev.timer_begin()
                    for d in dls:
                        ia.check(L.ifr_quant_gemm(dev.ctx, d, q.p, asc.p, gs.p, M, out.p, None), "gemm")
                    ms = dev.timer_end()
                    best = ms if best is None else min(best, ms)
                us = best * 1e3 / R
                byts = wb + M * K + M * 4 + M * N * 2
                ops = 2.0 * M * N * K
                res.append({"shape": name, "bits": bits, "M": M, "N": N, "K": K, "us": round(us, 3),
                            "GBps": round(byts / us / 1e3, 1), "hbm_frac": round(byts / us / 1e3 / 8000, 4),
                            "TOPS": round(ops / us / 1e6, 1), "mfma_frac": round(ops / us / 1e6 / 5000, 4),
                            "copies": R})
                log(f"cfg2 {name} W{bits} M={M}: {us:.2f} us, {byts / us / 1e3:.0f} GB/s, "
                    f"{ops / us / 1e6:.0f} TOPS")
            for d in dls:
                L.ifr_linear_free(dev.ctx, d)
            for b in (q, asc, gs, out):
                b.free()
    return res


def attn_cases(ia, cfg):
    """The attention sweep's cases: (name, decode-row KV lengths, prefill chunks (offset, rows))."""
    from intfer_amd import workloads as wl
    dec4 = [len(p) + 32 for p in wl.cfg4_requests(64, seed=4, vocab=cfg.vocab)]
    return [("cfg3", wl.cfg3_lengths(seed=3), [(0, 512), (1536, 512)]),
            ("prefill", [], [(1024, 512)]),
            ("c64_decode", dec4, []),
            ("c64_mixed", dec4, [(1024, 512)])]


def attn_case(ia, dev, spec):
    """One case of attn_sweep (NAME[:KV8[:REPS]]), launched REPS + 1 times
    back to back: the workload of a rocprofv3 kernel-trace of that case."""
    parts = spec.split(":")
    name = parts[0]
    kv_int8 = int(parts[1]) if len(parts) > 1 else 0
    reps = int(parts[2]) if len(parts) > 2 else 20
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = ia.SynthModel(cfg, seed=5)
    rng = np.random.default_rng(21)
    _, lens, chunks = next(c for c in attn_cases(ia, cfg) if c[0] == name)
    total = sum(lens) + sum(o + n for o, n in chunks)
    eng = ia.Engine(dev, model, max_seqs=len(lens) + len(chunks) + 1, max_seq_tokens=8192,
                    pool_tokens=total + 64 * (len(lens) + 4), kv_int8=kv_int8, max_rows=1200)
    seqs = []
    for n in lens + [o + m for o, m in chunks]:
        s = eng.seq_open()
        k = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
        eng.load_kv(s, k, k)
        seqs.append(s)
    rows = [(seqs[i], n - 1, 0, 0, 1) for i, n in enumerate(lens)]
    for j, (o, m) in enumerate(chunks):
        rows += [(seqs[len(lens) + j], o + p, 0, 1, 1) for p in range(m)]
    q = rng.standard_normal((len(rows), cfg.n_heads, cfg.head_dim), dtype=np.float32).astype(np.float16)
    for _ in range(reps + 1):
        eng.attention(0, rows, q)
    model.close()
    return {"metric": "attention case (rocprofv3 workload)", "case": name, "kv_int8": kv_int8,
            "rows": len(rows), "launches": reps + 1}


def attn_sweep(ia, dev, reps=10, splits=(0,)):
    """Joint ragged attention on one layer at the serve shapes: cfg3 (64
    decode rows, lognormal lengths, + two 512-row causal chunks), one
    512-row prefill chunk at offset 1024 alone, C=64 decode-only rows at the
    cfg4 context mix, and the same rows plus that chunk.  Durations come from HIP events on
    the engine stream around each launch (attention and combine separately)."""
    cfg = ia.default_cfg(layers=1, vocab=1024)
    model = ia.SynthModel(cfg, seed=5)
    rng = np.random.default_rng(21)
    cases = attn_cases(ia, cfg)
    res = []
    plan = [(kv, c, sp) for kv in (0, 1) for c in cases for sp in splits]
    for kv_int8, (name, lens, chunks), split in plan:
        if True:
            total = sum(lens) + sum(o + n for o, n in chunks)
            eng = ia.Engine(dev, model, max_seqs=len(lens) + len(chunks) + 1, max_seq_tokens=8192,
                            pool_tokens=total + 64 * (len(lens) + 4), kv_int8=kv_int8, max_rows=1200,
                            attn_split=split)
            seqs = []
            for n in lens + [o + m for o, m in chunks]:
                s = eng.seq_open()
                k = rng.standard_normal((1, n, cfg.n_kv, cfg.head_dim), dtype=np.float32)
                eng.load_kv(s, k, k)
                seqs.append(s)
            rows = [(seqs[i], n - 1, 0, 0, 1) for i, n in enumerate(lens)]
            for j, (o, m) in enumerate(chunks):
                rows += [(seqs[len(lens) + j], o + p, 0, 1, 1) for p in range(m)]
            q = rng.standard_normal((len(rows), cfg.n_heads, cfg.head_dim), dtype=np.float32).astype(np.float16)
            eng.attention(0, rows, q)  # warm code paths
            eng.set_timing(True)
            for _ in range(reps):
                eng.attention(0, rows, q)
            ms, n, b, f = eng.timing("attention")
            cms, cn, _, _ = eng.timing("combine")
            eng.set_timing(False)
            us = 1e3 * ms / n
            r = {"case": name, "kv_int8": kv_int8, "split": split, "rows": len(rows), "attn_us": round(us, 2),
                 "combine_us": round(1e3 * cms / cn, 2), "bytes": round(b / n),
                 "GBps": round(b / n / us / 1e3, 1), "hbm_frac": round(b / n / us / 1e3 / 8000, 4),
                 "TFLOPs": round(f / n / us / 1e6, 2)}
            res.append(r)
            log(f"attn {name} kv_int8={kv_int8} split={split}: {r}")
    model.close()
    return res


SHAPES_08B = [("qkv", 1024, 4096, False), ("o", 2048, 1024, False), ("gate_up", 1024, 3072, True),
              ("down", 3072, 1024, False)]
SHAPES_27B = [("qkv", 5120, 7168, False), ("o", 5120, 5120, False), ("gate_up", 5120, 17408, True),
              ("down", 17408, 5120, False)]


GEMM_CASES = {"qkv": SHAPES_08B[0], "o": SHAPES_08B[1], "gate_up": SHAPES_08B[2], "down": SHAPES_08B[3],
              "c5gu": SHAPES_27B[2], "c5down": SHAPES_27B[3]}


def gemm_case(ia, dev, spec, reps=20):
    """One W2A8 projection (codebook zeros, as the synthetic model) at one M
    through the engine's default launch shape, cache-cold (rotating weight
    copies over > 320 MB), `reps` passes: the workload of the counter runs
    under rocprofv3 --pmc."""
    import ctypes as C
    parts = spec.split(":")
    name, M = parts[0], int(parts[1])
    if len(parts) > 2:
        reps = int(parts[2])
    _, K, N, pair = GEMM_CASES[name]
    L = ia.lib()
    rng = np.random.default_rng(0)
    lins = [ia.make_linear(N, K, 2, rng) for _ in range(2 if pair else 1)]
    wb = sum(l.N * K * 2 // 8 + l.N * (K // 128) * 4 for l in lins)
    R = int(np.ceil(320e6 / wb))
    dls = []
    for _ in range(R):
        d = C.c_void_p()
        if pair:
            ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(lins[0].struct), C.byref(lins[1].struct),
                                              C.byref(d)), "upload")
        else:
            ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lins[0].struct), C.byref(d)), "upload")
        dls.append(d)
    q = dev.upload(rng.integers(-127, 128, size=((M + 15) // 16 * 16) * K, dtype=np.int8))
    asc = dev.upload(np.full(M, 1e-3, dtype=np.float32))
    gs = dev.upload(rng.integers(-2000, 2000, size=M * (K // 128)).astype(np.float32))
    out = dev.alloc(M * N * 2 * 2)
    fn = L.ifr_quant_gemm_swiglu if pair else L.ifr_quant_gemm
    extra = () if pair else (None,)
    dev.timer_begin()
    for _ in range(reps):
        for d in dls:
            ia.check(fn(dev.ctx, d, q.p, asc.p, gs.p, M, out.p, *extra), "gemm")
    ms = dev.timer_end()
    us = ms * 1e3 / (reps * R)
    ops = 2.0 * M * N * len(lins) * K
    byts = wb + M * K + M * 4 + M * N * len(lins) * 2
    for b in (q, asc, gs, out):
        b.free()
    for d in dls:
        L.ifr_linear_free(dev.ctx, d)
    return {"metric": "quant-GEMM case (cache-cold, default launch shape)", "shape": name, "M": M, "N": N,
            "K": K, "pair": pair, "launches": reps * R, "us": round(us, 2), "TOPS": round(ops / us / 1e6, 1),
            "mfma_frac": round(ops / us / 1e6 / 5000, 4), "GBps": round(byts / us / 1e3, 1),
            "hbm_frac": round(byts / us / 1e3 / 8000, 4)}


def f16_gemm(ia, dev, Ms=(1, 16, 576), reps=3, kind="f16"):
    """The FP16-activation dequant GEMM (ifr_quant_gemm_f16; kind "ga": the
    grouped-activation DPAS fold, ifr_quant_gemm_ga with 64-wide slices) on
    the plain 0.8B projections, cache-cold as in gemm_sweep (rotating weight
    copies over > 320 MB), HIP events around back-to-back launches, best of
    `reps`."""
    import ctypes as C
    L = ia.lib()
    rng = np.random.default_rng(0)
    res = []
    for name, K, N, pair in SHAPES_08B:
        if pair:
            continue
        lin = ia.make_linear(N, K, 2, rng)
        wb = lin.N * K * 2 // 8 + lin.N * (K // 128) * 4
        R = int(np.ceil(320e6 / wb))
        dls = []
        for _ in range(R):
            d = C.c_void_p()
            ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lin.struct), C.byref(d)), "upload")
            dls.append(d)
        for M in Ms:
            if kind == "ga":
                a = dev.upload(ia.atile(rng.integers(-127, 128, size=(M, K), dtype=np.int8)))
                asc = dev.upload((rng.random((M, K // 64)) * 0.05 + 1e-4).astype(np.float32))
                run = lambda d: L.ifr_quant_gemm_ga(dev.ctx, d, a.p, asc.p, M, 64, C.c_float(1.0), out.p)
                abytes = M * K + M * (K // 64) * 4
            else:
                a = dev.upload((rng.standard_normal((M, K)) * 2).astype(np.float16).view(np.uint16))
                run = lambda d: L.ifr_quant_gemm_f16(dev.ctx, d, a.p, M, C.c_float(1.0), out.p)
                abytes = M * K * 2
            out = dev.alloc(M * N * 2)
            best = None
            for _ in range(reps + 1):
                dev.timer_begin()
                for d in dls:
                    ia.check(run(d), kind + " gemm")
                ms = dev.timer_end()
                best = ms if best is None else min(best, ms)
            us = best * 1e3 / R
            byts = wb + abytes + M * N * 2
            res.append({"shape": name, "M": M, "us": round(us, 2), "GBps": round(byts / us / 1e3, 1),
                        "hbm_frac": round(byts / us / 1e3 / 8000, 4),
                        "TFLOPs": round(2.0 * M * N * K / us / 1e6, 2)})
            a.free()
            out.free()
            if kind == "ga":
                asc.free()
        for d in dls:
            L.ifr_linear_free(dev.ctx, d)
    return res


def gemm_variants(ia, dev, Ms=(128, 256, 576, 1024), bits=2, reps=3, shapes=SHAPES_08B, rotate_bytes=320e6,
                  rows=False):
    """Every launch shape of the quant GEMM on the four projection shapes
    (gate_up as the interleaved SwiGLU pair the forward runs), cache-cold as
    in gemm_sweep (rotate_bytes of distinct weight copies, above the 256 MB
    MALL); one line per (shape, M, variant).  With rotate_bytes = 100e6 the
    copies stay in the MALL but not in L2, as the 0.8B model's weights do in
    the serve load (28 layers x 4.4 MB, each touched once per iteration).
    rows: A also passed row-major (ifr_quant_gemm_rows; the weight stream
    stages its A rows from it at M <= 4)."""
    import ctypes as C
    L = ia.lib()
    rng = np.random.default_rng(0)
    res = []
    nv = L.ifr_quant_gemm_variants()
    Mmax = max(Ms)
    for name, K, N, pair in shapes:
        lins = [ia.make_linear(N, K, bits, rng) for _ in range(2 if pair else 1)]
        wb = sum(l.N * K * bits // 8 + l.N * (K // 128) * 4 for l in lins)
        R = int(np.ceil(rotate_bytes / wb))
        dls = []
        for _ in range(R):
            d = C.c_void_p()
            if pair:
                ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(lins[0].struct), C.byref(lins[1].struct),
                                                  C.byref(d)), "upload")
            else:
                ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lins[0].struct), C.byref(d)), "upload")
            dls.append(d)
        qrow = rng.integers(-127, 128, size=(Mmax, K), dtype=np.int8)
        q = dev.upload(ia.atile(qrow))
        qr = dev.upload(qrow)
        asc = dev.upload(np.full(Mmax, 1e-3, dtype=np.float32))
        gs = dev.upload(rng.integers(-2000, 2000, size=Mmax * (K // 128)).astype(np.float32))
        out = dev.alloc(Mmax * N * 2 * 2)

        def gemm(d, M, v):
            if rows:
                return L.ifr_quant_gemm_rows(dev.ctx, d, q.p, qr.p, asc.p, gs.p, M, out.p, v)
            return L.ifr_quant_gemm_variant(dev.ctx, d, q.p, asc.p, gs.p, M, out.p, v)
        for M in Ms:
            for v in range(nv):
                if gemm(dls[0], M, v) != 0:
                    continue
                best = None
                for _ in range(reps + 1):
                    dev.timer_begin()
                    for d in dls:
                        ia.check(gemm(d, M, v), "gemm")
                    ms = dev.timer_end()
                    best = ms if best is None else min(best, ms)
                us = best * 1e3 / R
                ops = 2.0 * M * N * len(lins) * K
                byts = wb + M * K + M * 4 + M * N * len(lins) * 2
                res.append({"shape": name, "M": M, "variant": v, "us": round(us, 2),
                            "TOPS": round(ops / us / 1e6, 1), "GBps": round(byts / us / 1e3, 1),
                            "hbm_frac": round(byts / us / 1e3 / 8000, 4)})
            row = [r for r in res if r["shape"] == name and r["M"] == M]
            b = min(row, key=lambda r: r["us"])
            log(f"{name} M={M}: best variant {b['variant']} {b['us']} us {b['TOPS']} TOPS "
                f"{b['GBps']} GB/s; " +
                " ".join(f"v{r['variant']}:{r['us']}" for r in row))
        for d in dls:
            L.ifr_linear_free(dev.ctx, d)
        for b in (q, qr, asc, gs, out):
            b.free()
    return res


def decode_gemm_brief(ia, dev, reps=3):
    """The W2A8 decode GEMM (M = 1, the library's default launch shape),
    cache-cold as in gemm_sweep: the 0.8B gate/up pair and the 27B-class
    gate/up pair and down projection (the largest weight streams).  us: A in
    the A-tile layout (ifr_quant_gemm / ifr_quant_gemm_swiglu, what the
    engine's forward passes); us_rows: A also row-major
    (ifr_quant_gemm_rows)."""
    import ctypes as C
    L = ia.lib()
    rng = np.random.default_rng(1)
    res = []
    for name, K, N, pair in (("gate_up_0.8b", 1024, 3072, True), ("gate_up_27b", 5120, 17408, True),
                             ("down_27b", 17408, 5120, False)):
        lins = [ia.make_linear(N, K, 2, rng) for _ in range(2 if pair else 1)]
        wb = sum(l.N * K * 2 // 8 + l.N * (K // 128) * 4 for l in lins)
        R = int(np.ceil(320e6 / wb))
        dls = []
        for _ in range(R):
            d = C.c_void_p()
            if pair:
                ia.check(L.ifr_linear_upload_pair(dev.ctx, C.byref(lins[0].struct), C.byref(lins[1].struct),
                                                  C.byref(d)), "upload")
            else:
                ia.check(L.ifr_linear_upload(dev.ctx, C.byref(lins[0].struct), C.byref(d)), "upload")
            dls.append(d)
        qrow = rng.integers(-127, 128, size=(1, K), dtype=np.int8)
        q = dev.upload(ia.atile(qrow))
        qr = dev.upload(qrow)
        asc = dev.upload(np.full(16, 1e-3, dtype=np.float32))
        gs = dev.upload(rng.integers(-2000, 2000, size=16 * (K // 128)).astype(np.float32))
        out = dev.alloc(16 * N * 2 * 2)

        def timed(rows):
            best = None
            for _ in range(reps + 1):
                dev.timer_begin()
                for d in dls:
                    if rows:
                        ia.check(L.ifr_quant_gemm_rows(dev.ctx, d, q.p, qr.p, asc.p, gs.p, 1, out.p, -1), "rows")
                    elif pair:
                        ia.check(L.ifr_quant_gemm_swiglu(dev.ctx, d, q.p, asc.p, gs.p, 1, out.p), "swiglu")
                    else:
                        ia.check(L.ifr_quant_gemm(dev.ctx, d, q.p, asc.p, gs.p, 1, out.p, None), "gemm")
                ms = dev.timer_end()
                best = ms if best is None else min(best, ms)
            return best * 1e3 / R
        # the row-major copy is read only by the weight stream (K >= 4096);
        # on the small shapes both entries run the same kernel and a
        # back-to-back loop of 3 us launches times the host calls
        us = timed(False)
        us_rows = timed(True) if K >= 4096 else None
        byts = wb + K + 4 + N * 2
        res.append({"shape": name, "M": 1, "K": K, "N": N * len(lins), "weight_MB": round(wb / 1e6, 2),
                    "us": round(us, 2), "GBps": round(byts / us / 1e3, 1),
                    "hbm_frac": round(byts / us / 1e3 / 8000, 4),
                    "us_rows": round(us_rows, 2) if us_rows else None,
                    "hbm_frac_rows": round(byts / us_rows / 1e3 / 8000, 4) if us_rows else None})
        log(f"decode GEMM {name} M=1: {us:.2f} us, {byts / us / 1e3:.0f} GB/s" +
            (f"; A row-major {us_rows:.2f} us" if us_rows else ""))
        for d in dls:
            L.ifr_linear_free(dev.ctx, d)
        for b in (q, qr, asc, gs, out):
            b.free()
    return res


def _read(path, default=""):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return default


def _cpulist(text):
    cpus = set()
    for part in text.split(","):
        if "-" in part:
            lo, hi = part.split("-")
            cpus.update(range(int(lo), int(hi) + 1))
        elif part.strip():
            cpus.add(int(part))
    return cpus


def gpu_numa_node():
    """NUMA node of the GPU this process sees: the render node under /dev/dri
    (the container shows only its own card) mapped to its PCI device."""
    try:
        nodes = sorted(n for n in os.listdir("/dev/dri") if n.startswith("renderD"))
    except OSError:
        return None
    found = set()
    for n in nodes:
        dev = f"/sys/class/drm/{n}/device"
        if _read(dev + "/vendor") != "0x1002":
            continue
        v = _read(dev + "/numa_node", "-1")
        if v.lstrip("-").isdigit():
            found.add(int(v))
    # -1: the platform reports no NUMA locality for the device
    return found.pop() if len(found) == 1 else None


def bind_host_cpus():
    """Pin this process (and the CPU path's OpenMP threads it starts later) to
    the CPUs of the GPU's NUMA node that it may use, and describe the host:
    CPU model, nproc, the CPU set, its physical cores and the thread count."""
    allowed = os.sched_getaffinity(0)
    node = gpu_numa_node()
    bound = False
    if node is not None and node >= 0:
        mine = _cpulist(_read(f"/sys/devices/system/node/node{node}/cpulist")) & allowed
        if mine:
            os.sched_setaffinity(0, mine)
            allowed, bound = mine, True
    cores = {(_read(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id"),
              _read(f"/sys/devices/system/cpu/cpu{c}/topology/core_id")) for c in allowed}
    model_name = ""
    for ln in _read("/proc/cpuinfo").splitlines():
        if ln.startswith("model name"):
            model_name = ln.split(":", 1)[1].strip()
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", len(allowed)))
    return {"host_cpu": model_name, "host_nproc": os.cpu_count(), "gpu_numa_node": node,
            "numa_bound": bound, "cpus": len(allowed), "physical_cores": len(cores),
            "omp_threads": threads, "cores": min(threads, len(allowed))}


def measure_peaks(ia, dev):
    """Measured denominators next to the nominal ones: a streaming read of a
    2 GiB buffer (8x the 256 MB Infinity Cache; each 16-byte word read once
    per launch, 10 launches), and back-to-back independent int8 / fp16 MFMAs
    in two waves per SIMD (ifr_peak_read / ifr_peak_mfma, HIP events)."""
    import ctypes as C
    L = ia.lib()
    n = 2 << 30
    buf = dev.zeros(n)
    gbps, i8, f16 = C.c_double(), C.c_double(), C.c_double()
    ia.check(L.ifr_peak_read(dev.ctx, buf.p, C.c_size_t(n), 10, C.byref(gbps)), "ifr_peak_read")
    buf.free()
    ia.check(L.ifr_peak_mfma(dev.ctx, 0, 4000, 5, C.byref(i8)), "ifr_peak_mfma int8")
    ia.check(L.ifr_peak_mfma(dev.ctx, 1, 4000, 5, C.byref(f16)), "ifr_peak_mfma fp16")
    return {"hbm_read_GBps": round(gbps.value, 1), "int8_TOPS": round(i8.value, 1),
            "fp16_TFLOPs": round(f16.value, 1),
            "nominal": {"hbm_GBps": HBM_PEAK / 1e9, "int8_TOPS": INT8_PEAK / 1e12, "fp16_TFLOPs": FP16_PEAK / 1e12},
            "method": "read: 2 GiB buffer, nontemporal 16-byte loads, 10 launches; MFMA: 8 independent "
                      "accumulators per wave, 2 waves per SIMD, 4000 rounds, 5 launches (HIP events)"}


def with_measured(r, peaks):
    """Add frac_measured (achieved / the measured peak of the same unit) to a roofline dict."""
    if not peaks or not r or r.get("achieved") is None:
        return r
    if r.get("unit") == "GB/s":
        r["frac_measured"] = round(r["achieved"] / peaks["hbm_read_GBps"], 4)
    elif r.get("unit") == "TFLOP/s":
        meas = peaks["int8_TOPS"] if r.get("peak") == INT8_PEAK / 1e12 else peaks["fp16_TFLOPs"]
        r["frac_measured"] = round(r["achieved"] / meas, 4)
    return r


def cpu_baseline(ia, model, cfg):
    """Reference CPU path on a bounded sample with the load's per-output-token
    mix: 4 decode rows at the load's mean context (1088) + one 66-row prefill
    chunk at offset 512 (each request of the load prefills ~16.5 tokens per
    output token).  cpu tok/s = decode rows / iteration time."""
    from oracle import pyoracle as po
    host = bind_host_cpus()
    ora = po.OracleEngine(model, mode=1, max_seqs=8)
    rng = np.random.default_rng(0)
    ctx, D, P, off = 1088, 4, 66, 512
    seqs = []
    for _ in range(D):
        s = ora.seq_open()
        k = rng.standard_normal((cfg.layers, ctx, cfg.n_kv * cfg.head_dim), dtype=np.float32)
        ora.set_kv(s, k, k)
        seqs.append(s)
    sp = ora.seq_open()
    kp = rng.standard_normal((cfg.layers, off, cfg.n_kv * cfg.head_dim), dtype=np.float32)
    ora.set_kv(sp, kp, kp)
    rows = [(s, ctx, int(rng.integers(0, cfg.vocab)), 0, 1) for s in seqs]
    rows += [(sp, off + i, int(rng.integers(0, cfg.vocab)), 1, 0) for i in range(P)]
    t0 = time.perf_counter()
    ora.forward(rows)
    dt = time.perf_counter() - t0
    ora.close()
    return {"value": D / dt, "unit": "tok/s", "cores": host["cores"], "kind": "port", **host,
            "sample": f"one mixed iteration of the 28-layer f32 CPU path: {D} decode rows at "
                      f"context {ctx} + a {P}-row prefill chunk at offset {off} "
                      f"(the load's ~16.5 prefill tokens per output token); {dt:.1f} s; "
                      "the full plan (bench.py --cpu-full) times cfg1, cfg2 and cfg4 C=1 / 4"}


def cpu_full(ia, wl):
    """The CPU-baseline plan on the host cores: the reference CpuBackend path
    restated (oracle f32 mode: weights dequantized once to fp32, OpenMP row
    dot above M*N >= 2048, single-threaded host attention, fp32 tied lm_head).
      cfg1  one mixed iteration (4 decode rows at contexts 17 / 133 / 512 /
            1000 + a 60-row prefill chunk), best of 2
      cfg2  the fp32-dequant dot of every 0.8B GEMM shape at M = 1 .. 1024
      cfg4  decode iterations at C = 1 and C = 4 (each sequence's context
            = its cfg4 prompt, KV seeded N(0,1), one row per sequence per
            iteration, argmax fed back), 8 iterations each
      load  C = 1, 4, 64 loads extrapolated from those: prompt tokens x the
            prefill cost per row (cfg1 minus its decode rows) + C x 64 decode
            rows x the decode cost per row at C = 4"""
    from oracle import pyoracle as po
    host = bind_host_cpus()
    cfg = ia.default_cfg()
    log("cpu-full: building the synthetic 0.8B-class INT2 model")
    model = ia.SynthModel(cfg, seed=11, bits=2)
    out = {"metric": "reference CPU path (f32 CpuBackend restatement) on the host cores", "kind": "port",
           **host}
    ora = po.OracleEngine(model, mode=1, max_seqs=8)
    # cfg1
    w = wl.cfg1(cfg, seed=1)
    times = []
    for _ in range(2):
        dec = []
        for (k, v) in w.kv:
            s = ora.seq_open()
            ora.set_kv(s, k.reshape(cfg.layers, k.shape[1], -1), v.reshape(cfg.layers, v.shape[1], -1))
            dec.append(s)
        pre = ora.seq_open()
        t0 = time.perf_counter()
        ora.forward(wl.cfg1_rows(w, dec, pre))
        times.append(time.perf_counter() - t0)
        for s in dec + [pre]:
            ora.seq_close(s)
    t_cfg1 = min(times)
    out["cfg1"] = {"iteration_s": [round(t, 3) for t in times], "rows": 64}
    log(f"cpu-full: cfg1 iteration {t_cfg1:.2f} s")
    # cfg2: fp32-dequant dot per shape and M (weights dequantized beforehand)
    O = po.oracle()
    rng = np.random.default_rng(2)
    g2 = []
    for name, K, N in (("qkv", 1024, 4096), ("o", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)):
        W = rng.standard_normal((N, K), dtype=np.float32)
        for M in (1, 8, 16, 64, 256, 1024):
            X = rng.standard_normal((M, K), dtype=np.float32)
            Y = np.empty((M, N), np.float32)
            t0 = time.perf_counter()
            O.or_gemm_f32(po.ptr(W), po.ptr(X), po.ptr(Y), M, N, K)
            dt = time.perf_counter() - t0
            g2.append({"shape": name, "M": M, "N": N, "K": K, "ms": round(1e3 * dt, 3),
                       "GFLOPs": round(2.0 * M * N * K / dt / 1e9, 2),
                       "weight_GBps": round(4.0 * N * K / dt / 1e9, 2)})
    out["cfg2"] = g2
    log("cpu-full: cfg2 done")
    # cfg4 decode windows
    dec_row = {}
    for C in (1, 4):
        prompts = wl.cfg4_requests(C, seed=4, vocab=cfg.vocab)
        seqs, pos, tok = [], [], []
        for p in prompts:
            s = ora.seq_open()
            k = rng.standard_normal((cfg.layers, len(p), cfg.n_kv * cfg.head_dim), dtype=np.float32)
            ora.set_kv(s, k, k)
            seqs.append(s)
            pos.append(len(p))
            tok.append(int(p[-1]))
        it = []
        for _ in range(8):
            rows = [(s, q, t, 0, 1) for s, q, t in zip(seqs, pos, tok)]
            t0 = time.perf_counter()
            best = ora.forward(rows)
            it.append(time.perf_counter() - t0)
            pos = [q + 1 for q in pos]
            tok = [int(b) for b in best]
        for s in seqs:
            ora.seq_close(s)
        t_it = sum(it) / len(it)
        dec_row[C] = t_it / C
        out[f"cfg4_c{C}_decode"] = {"iterations": len(it), "iteration_s_mean": round(t_it, 4),
                                    "tok_s": round(C / t_it, 3),
                                    "contexts": [len(p) for p in prompts]}
        log(f"cpu-full: C={C} decode {t_it:.3f} s per iteration")
    ora.close()
    # extrapolated loads
    pre_row = max(t_cfg1 - 4 * dec_row[4], 0.0) / 60
    loads = {}
    for C in (1, 4, 64):
        ptoks = sum(len(p) for p in wl.cfg4_requests(C, seed=4, vocab=cfg.vocab))
        t = ptoks * pre_row + C * 64 * dec_row[4 if C >= 4 else 1]
        loads[f"c{C}"] = {"prompt_tokens": ptoks, "load_s": round(t, 1), "tok_s": round(C * 64 / t, 4)}
    out["cfg4_loads_extrapolated"] = {"prefill_s_per_row": round(pre_row, 5),
                                      "decode_s_per_row": {str(k): round(v, 5) for k, v in dec_row.items()},
                                      **loads}
    model.close()
    print(json.dumps(out))
    return 0


def cfg5_bench(ia, a):
    """cfg5: one mixed iteration of the 27B-class model (hidden 5120, 64
    layers, 40 q / 8 kv heads, FFN 17408, seeded 70 / 30 INT2 / INT4 split,
    INT8 KV): 48 decode sequences with contexts U[512, 4096] -- 16 of them
    speculating with 4 n-gram drafts each, so their decode row becomes a
    5-row verify group -- plus one 2048-token prefill chunk: M = 32 + 80 +
    2048 = 2160.  The contexts are built by real prefill forwards of
    uniform random tokens; after every iteration the sequences are cut back
    (seq_truncate) so each timed iteration runs the same rows."""
    from intfer_amd import workloads as wl  # noqa: F401  (same seeded style as the other configs)
    cfg = ia.default_cfg(hidden=5120, layers=64, n_heads=40, n_kv=8, inter=17408)
    t0 = time.perf_counter()
    model = ia.SynthModel(cfg, seed=27, bits=0)
    log(f"27B-class synthetic model built in {time.perf_counter() - t0:.1f} s")
    dev = ia.Device(0)
    rng = np.random.default_rng(5)
    ctx = rng.integers(512, 4097, size=48).tolist()
    spec = set(rng.choice(48, size=16, replace=False).tolist())
    cap = 4224
    t0 = time.perf_counter()
    eng = ia.Engine(dev, model, max_seqs=50, max_seq_tokens=cap, pool_tokens=sum(ctx) + 48 * 64 + 2048 + 4096,
                    kv_int8=1, max_rows=2304)
    # device bytes of the quantized linears (codes + fp16 scale/zero pairs), exact per tensor
    wbytes = 0.0
    for l in range(cfg.layers):
        lw = model.layer(l)
        for nm in ("q", "k", "v", "o", "gate", "up", "down"):
            t = getattr(lw, nm)
            wbytes += t.N * t.K * t.bits / 8 + t.N * (t.K // 128) * 4
    model.close()
    log(f"model loaded in {time.perf_counter() - t0:.1f} s")
    V = cfg.vocab
    seqs = []
    t0 = time.perf_counter()
    for n in ctx:
        s = eng.seq_open()
        toks = rng.integers(0, V, size=n).tolist()
        for c0 in range(0, n, 2048):
            eng.forward([(s, p, toks[p], ia.ROW_PREFILL, 0) for p in range(c0, min(n, c0 + 2048))])
        seqs.append(s)
    log(f"48 contexts ({sum(ctx)} tokens) prefilled in {time.perf_counter() - t0:.1f} s")
    pre = eng.seq_open()
    it_toks = rng.integers(0, V, size=48 * 5 + 2048).tolist()
    rows = []
    k = 0
    for j, s in enumerate(seqs):
        if j in spec:
            for d in range(5):
                rows.append((s, ctx[j] + d, it_toks[k], ia.ROW_VERIFY, 1))
                k += 1
        else:
            rows.append((s, ctx[j], it_toks[k], ia.ROW_DECODE, 1))
            k += 1
    for p in range(2048):
        rows.append((pre, p, it_toks[k], ia.ROW_PREFILL, int(p == 2047)))
        k += 1
    arr = ia.rows_array(rows)
    M = len(rows)

    def once():
        eng.forward(arr)
        for j, s in enumerate(seqs):
            eng.seq_truncate(s, ctx[j])
        eng.seq_truncate(pre, 0)

    for _ in range(a.warmup):
        once()
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        once()
    dev.sync()
    ms = 1e3 * (time.perf_counter() - t0) / a.steps
    # roofline of the iteration: t = max(bytes / HBM peak, int8 ops / int8 peak + attention flops / fp16 peak)
    H, L, nq, nkv, hd, F = cfg.hidden, cfg.layers, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.inter
    per_layer = H * (nq * hd + 2 * nkv * hd) + nq * hd * H + H * 2 * F + F * H
    nwant = sum(r[4] for r in rows)
    lm_bytes = V * H + V * 2
    kv_tok = L * nkv * hd * 2 * (1 + 2 / hd)      # int8 K+V + fp16 scale per (token, kv head)
    vis = [r[1] + 1 for r in rows]                 # causal: a row sees pos + 1 tokens
    kv_bytes = sum(ctx) * kv_tok + 2048 * kv_tok   # each sequence's cache read once per layer
    ops = 2.0 * M * L * per_layer + 2.0 * nwant * V * H
    flops = sum(4.0 * nq * hd * v for v in vis) * L
    t_hbm = (wbytes + lm_bytes + kv_bytes) / HBM_PEAK
    t_mfma = ops / INT8_PEAK + flops / FP16_PEAK
    t_roof = max(t_hbm, t_mfma)
    out = {"metric": "cfg5 27B-class mixed iteration (1 GPU)", "value": round(M / ms * 1e3, 1),
           "unit": "rows/s", "ms_per_iteration": round(ms, 3), "steps": a.steps, "warmup": a.warmup,
           "higher_is_better": True, "dtype": "int8 x int2/int4 -> int32 GEMM, int8 KV",
           "data": "synthetic (seeded random-init weights, uniform token ids)",
           "config": {"workload": "cfg5: 32 decode + 16 x (1 + 4 drafts) verify + 2048 prefill rows",
                      "M": M, "contexts_mean": round(float(np.mean(ctx)), 1)},
           "roofline": {"bound": "mfma" if t_mfma >= t_hbm else "hbm",
                        "t_roof_ms": round(1e3 * t_roof, 3), "t_hbm_ms": round(1e3 * t_hbm, 3),
                        "t_mfma_ms": round(1e3 * t_mfma, 3), "frac": round(1e3 * t_roof / ms, 4),
                        "int8_ops": ops, "attn_flops": flops,
                        "bytes": wbytes + lm_bytes + kv_bytes}}
    if not a.no_roofline:
        eng.set_timing(True)
        once()
        stats = {k2: eng.timing(k2) for k2 in KERNELS}
        eng.set_timing(False)
        out["kernels_ms"] = {k2: round(v[0], 3) for k2, v in stats.items() if v[1]}
        g = [stats[k2] for k2 in GEMMS]
        gms = sum(x[0] for x in g)
        out["quant_gemm"] = {"ms": round(gms, 3), "TOPS": round(sum(x[3] for x in g) / gms / 1e9, 1),
                             "frac_int8_peak": round(sum(x[3] for x in g) / gms / 1e9 / 5000, 4)}
    print(json.dumps(out))
    dev.close()
    return 0


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported "
              "(the path shards as independent data-parallel engines, one per GPU)",
              file=sys.stderr)
        return 2
    import intfer_amd as ia
    from intfer_amd import workloads as wl

    if a.copy_calib:
        import ctypes as C
        dev = ia.Device(0)
        n = 1 << 30
        src, dst = dev.zeros(n), dev.alloc(n)
        dev.timer_begin()
        for _ in range(8):
            ia.check(ia.lib().ifr_d2d(dev.ctx, dst.p, src.p, C.c_size_t(n)), "ifr_d2d")
        ms = dev.timer_end()
        print(json.dumps({"metric": "device copy 1 GiB x 8", "bytes_read_per_copy": n,
                          "bytes_written_per_copy": n, "GBps": round(2 * 8 * n / ms / 1e6, 1)}))
        dev.close()
        return 0
    if a.peaks:
        dev = ia.Device(0)
        print(json.dumps({"metric": "device peaks (measured)", **measure_peaks(ia, dev)}))
        dev.close()
        return 0
    if a.cfg5:
        return cfg5_bench(ia, a)
    if a.cpu_full:
        return cpu_full(ia, wl)
    if a.f16_gemm:
        dev = ia.Device(0)
        print(json.dumps({"metric": "FP16-activation dequant GEMM (reference default linear), cache-cold",
                          "unit": "us", "results": f16_gemm(ia, dev)}))
        dev.close()
        return 0
    if a.ga_gemm:
        dev = ia.Device(0)
        print(json.dumps({"metric": "grouped-activation (GA64) DPAS-fold GEMM, cache-cold",
                          "unit": "us", "results": f16_gemm(ia, dev, kind="ga")}))
        dev.close()
        return 0
    if a.gemm_case:
        dev = ia.Device(0)
        res = gemm_case(ia, dev, a.gemm_case)
        print(json.dumps(res))
        dev.close()
        return 0
    if a.attn_case:
        dev = ia.Device(0)
        print(json.dumps(attn_case(ia, dev, a.attn_case)))
        dev.close()
        return 0
    if a.attn_sweep:
        dev = ia.Device(0)
        res = attn_sweep(ia, dev, splits=tuple(int(x) for x in a.attn_splits.split(",")))
        print(json.dumps({"metric": "ragged joint attention sweep (1 layer)", "unit": "GB/s",
                          "results": res}))
        dev.close()
        return 0
    if a.gemm_variants or a.gemm_variants_27b or a.gemm_decode_27b or a.gemm_decode:
        dev = ia.Device(0)
        if a.gemm_variants:
            res = gemm_variants(ia, dev, Ms=tuple(int(m) for m in a.gemm_ms.split(",")),
                                rotate_bytes=100e6 if a.gemm_mall else 320e6)
        elif a.gemm_decode:
            res = gemm_variants(ia, dev, Ms=(1, 8, 16), shapes=SHAPES_08B, reps=3)
        elif a.gemm_variants_27b:
            res = gemm_variants(ia, dev, Ms=(512, 2160), shapes=SHAPES_27B, reps=2)
        else:
            res = gemm_variants(ia, dev, Ms=(1, 8, 16), shapes=SHAPES_27B, reps=3)
            res += [dict(r, A="rows") for r in gemm_variants(ia, dev, Ms=(1, 4), shapes=SHAPES_27B, reps=3,
                                                               rows=True)]
        print(json.dumps({"metric": "quant-GEMM launch shapes (cache-cold)", "unit": "us", "results": res}))
        dev.close()
        return 0
    if a.gemm_sweep:
        dev = ia.Device(0)
        res = gemm_sweep(ia, dev)
        dec = [r for r in res if r["M"] <= 16]
        print(json.dumps({"metric": "cfg2 quant-GEMM sweep (cache-cold, rotating weights > MALL)",
                          "unit": "GB/s", "decode_best_hbm_frac": max(r["hbm_frac"] for r in dec),
                          "results": res}))
        dev.close()
        return 0

    cfg = ia.default_cfg()
    log("building the synthetic 0.8B-class INT2 model")
    model = ia.SynthModel(cfg, seed=11, bits=2)
    dev = ia.Device(0)
    C, max_new, chunk = a.concurrency, a.max_new, a.chunk
    cap = 2176
    eng = ia.Engine(dev, model, max_seqs=C, max_seq_tokens=cap, pool_tokens=C * cap,
                    kv_int8=a.kv_int8, max_rows=64 + chunk, attn_split=a.attn_split, lanes=a.lanes)
    prompts = wl.cfg4_requests(C, seed=4, vocab=cfg.vocab)
    log(f"C={C} prompts: mean {np.mean([len(p) for p in prompts]):.0f} tokens, max_new {max_new}")
    for w in range(a.warmup):
        dt, toks, iters, rows, _ = run_load(ia, eng, prompts, max_new, chunk)
        log(f"warmup {w}: {dt:.3f} s, {iters} iterations, {toks / dt:.0f} tok/s")
    dev.sync()
    total_t = 0.0
    total_tok = 0
    lat = []
    iters_total = 0
    for s in range(a.steps):
        dt, toks, iters, rows, done = run_load(ia, eng, prompts, max_new, chunk)
        dev.sync()
        total_t += dt
        total_tok += toks
        lat += done
        iters_total += iters
        log(f"step {s}: {dt:.3f} s, {iters} iterations, {rows} rows, {toks / dt:.0f} tok/s")
    value = total_tok / total_t
    out = {
        "metric": "output tok/s @C=64 0.8B-INT2 (1 GPU); quant-GEMM HBM GB/s as % of peak",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1e3 * total_t / a.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8xint2->int32 GEMM, fp16 KV" if not a.kv_int8 else "int8xint2->int32 GEMM, int8 KV",
        "data": "synthetic (seeded random-init weights and uniform token-id prompts)",
        "config": {"workload": "cfg4 serve load C=64: prompts U[64,2048], max_new 64, greedy, "
                               "chunk 512, round-robin", "concurrency": C,
                   "requests_per_step": C, "req_per_s": round(C * a.steps / total_t, 3),
                   "p50_latency_s": round(pct(lat, 50), 4), "p99_latency_s": round(pct(lat, 99), 4),
                   "iterations_per_step": iters_total // a.steps},
    }
    if not a.no_roofline:
        rec = []
        eng.set_timing(True)
        dt, toks, iters, rows, _ = run_load(ia, eng, prompts, max_new, chunk, record=rec)
        stats = {k: eng.timing(k) for k in KERNELS}
        eng.set_timing(False)
        dom = max(KERNELS, key=lambda k: stats[k][0])
        out["roofline"] = kernel_roofline(dom, stats[dom], a.kv_int8)
        out["kernels"] = {k: kernel_roofline(k, v, a.kv_int8, brief=True)
                          for k, v in stats.items() if v[1]}
        g = [stats[k] for k in GEMMS]
        out["quant_gemm"] = kernel_roofline("qgemm", tuple(sum(x[i] for x in g) for i in range(4)),
                                            a.kv_int8, brief=True)
        out["quant_gemm"]["note"] = ("all in-load W2A8 GEMMs (mixed M); the cache-cold cfg2 sweep "
                                     "(bench.py --gemm-sweep) reports decode-shape HBM GB/s")
        kv_elem = 1 if a.kv_int8 else 2
        H, L = cfg.hidden, cfg.layers
        per_layer = (H * (cfg.n_heads * cfg.head_dim + 2 * cfg.n_kv * cfg.head_dim) +
                     cfg.n_heads * cfg.head_dim * H + H * 2 * cfg.inter + cfg.inter * H)
        wbytes = L * per_layer * 2 / 8 + L * per_layer / 128 * 4
        lm_bytes = cfg.vocab * H + cfg.vocab * 2
        t_roof, dec = serve_roofline(cfg, wbytes, lm_bytes, rec, kv_elem)
        roof_tok_s = C * max_new / t_roof
        out["serve_roofline"] = {"roofline_tok_s": round(roof_tok_s, 1),
                                 "achieved_tok_s": round(value, 1),
                                 "frac": round(value / roof_tok_s, 4),
                                 "decode_rows": dec, "iterations": len(rec)}
        log(f"timing pass: {dt:.3f} s; dominant {dom} {stats[dom][0]:.1f} ms; roofline tok/s {roof_tok_s:.0f}")
        # the same fractions against the peaks measured on this device
        peaks = measure_peaks(ia, dev)
        out["peaks"] = peaks
        with_measured(out["roofline"], peaks)
        with_measured(out["quant_gemm"], peaks)
        for v in out["kernels"].values():
            with_measured(v, peaks)
        t_meas, _ = serve_roofline(cfg, wbytes, lm_bytes, rec, kv_elem,
                                   bw=peaks["hbm_read_GBps"] * 1e9, i8=peaks["int8_TOPS"] * 1e12,
                                   f16=peaks["fp16_TFLOPs"] * 1e12)
        out["serve_roofline"]["frac_measured"] = round(value / (C * max_new / t_meas), 4)
    if not a.no_packed:
        # the same load with the chunk budget filled from several queued
        # prompts (pack_prefill; the reference fills it from the head only):
        # same token streams, fewer iterations; reported beside `value`
        run_load(ia, eng, prompts, max_new, chunk, pack=1)
        dev.sync()
        dt, toks, iters, rows, done = run_load(ia, eng, prompts, max_new, chunk, pack=1)
        dev.sync()
        out["packed_prefill"] = {"value": round(toks / dt, 2), "unit": "tok/s", "iterations": iters,
                                 "ms_per_step": round(1e3 * dt, 3), "p50_latency_s": round(pct(done, 50), 4),
                                 "p99_latency_s": round(pct(done, 99), 4),
                                 "note": "scheduler option pack_prefill=1 (not the reference policy)"}
        log(f"packed prefill: {dt:.3f} s, {iters} iterations, {toks / dt:.0f} tok/s")
    if not a.no_gemm:
        out["decode_gemm"] = {
            "note": "W2A8 decode GEMM at M=1, cache-cold (rotating weight copies > MALL), HIP events "
                    "around back-to-back launches (each includes the ~2.3 us launch floor); us: A-tile "
                    "layout (the engine's path), us_rows: A also row-major (ifr_quant_gemm_rows)",
            "results": decode_gemm_brief(ia, dev)}
    if not a.no_cpu:
        log("timing the reference CPU path on a bounded sample")
        out["cpu_baseline"] = cpu_baseline(ia, model, cfg)
    print(json.dumps(out))
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
