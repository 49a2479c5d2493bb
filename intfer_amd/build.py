"""Build the gfx950 shared library intfer_amd/libintfer_amd.so with hipcc.

Every source is compiled for gfx950 only, with fused multiply-add contraction
off (each fused operation in the kernels is an explicit fmaf, so results do
not depend on the compiler's contraction choices) and packed-fp32 codegen off.
Objects go to intfer_amd/_build/ (git-ignored); the .so is written in-tree so
it travels with the repository snapshot.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libintfer_amd.so"

# (source, extra flags, object name): qgemm.hip compiles once per code width
# (its kernels) and once without (packing and dispatch), in parallel.
SOURCES = [("qgemm.hip", [], "qgemm"),
           ("qgemm.hip", ["-DIFR_QGEMM_BITS=2"], "qgemm_b2"),
           ("qgemm.hip", ["-DIFR_QGEMM_BITS=4"], "qgemm_b4"),
           ("qgemm.hip", ["-DIFR_QGEMM_BITS=8"], "qgemm_b8"),
           ("rows.hip", [], "rows"), ("attn.hip", [], "attn"), ("lmhead.hip", [], "lmhead"),
           ("engine.cpp", [], "engine"), ("sched.cpp", [], "sched"), ("synth.cpp", [], "synth"),
           ("intfer_file.cpp", [], "intfer_file"), ("serve.cpp", [], "serve"),
           ("sample.cpp", [], "sample"), ("qgemm_f16.hip", [], "qgemm_f16"),
           ("qgemm_ga.hip", [], "qgemm_ga"), ("peak.hip", [], "peak")]
SERVE_BIN = HERE / "intfer_serve"  # the --serve command line (serve_main.cpp)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3", "-fPIC", "-std=c++17", "--offload-arch=gfx950", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-value", "-Wno-unused-result",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


# MFMA results of the GEMMs feed VALU work at once (the per-group fold), and
# attention rescales its O accumulators between MFMAs, so both keep MFMA
# results in VGPRs instead of round-tripping through AGPRs; the peak
# microbenchmark too (its accumulators otherwise shuffle between AGPRs and
# VGPRs every round, which serializes the MFMA pipe).
EXTRA = {"qgemm.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"], "attn.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"],
         "peak.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"]}


def _compile(item) -> Path:
    src, defs, name = item
    s = CSRC / src
    o = BUILD / (name + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), *defs, "-x", "hip", "-c", str(s), "-o", str(o)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    # hipcc's host pass warns about the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in r.stderr.splitlines() if noise not in ln and ln.strip()]
    if msgs:
        sys.stderr.write(f"[{src}]\n" + "\n".join(msgs) + "\n")
    return o


def build(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    # The command line links the library in place (found next to itself).
    tmpb = SERVE_BIN.with_suffix(".tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}", str(CSRC / "serve_main.cpp"),
           f"-L{HERE}", "-lintfer_amd", "-Wl,-rpath,$ORIGIN", "-o", str(tmpb)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"intfer_serve link failed:\n{r.stderr[-4000:]}")
    os.replace(tmpb, SERVE_BIN)
    return LIB


if __name__ == "__main__":
    print(build())
