"""Build the CPU emulation of the library (test infrastructure only).

Compiles the unmodified kernel and engine sources of intfer_amd/csrc for the
host with clang++ and AddressSanitizer, against tests/hipemu/hip/hip_runtime.h
instead of the HIP runtime, into tests/hipemu/_build/libintfer_emu.so.  Two
mechanical rewrites are applied to copies of the sources first, because the
host compiler has no equivalent syntax:
  * `extern __shared__ T name[];`  ->  a pointer to the launch's dynamic LDS
  * the AMDGPU register constraint "+v" of the empty asm pins -> "+x"
The result is loaded only by tests/hipemu/runner.py, in a subprocess that
preloads the ASan runtime.  The product library is never replaced by it.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
CSRC = ROOT / "intfer_amd" / "csrc"
BUILD = HERE / "_build"
SRC = BUILD / "src"
LIB = BUILD / "libintfer_emu.so"
CLANG = "/opt/rocm/llvm/bin/clang++"

UNITS = [("qgemm.hip", [], "qgemm"),
         ("qgemm.hip", ["-DIFR_QGEMM_BITS=2"], "qgemm_b2"),
         ("qgemm.hip", ["-DIFR_QGEMM_BITS=4"], "qgemm_b4"),
         ("qgemm.hip", ["-DIFR_QGEMM_BITS=8"], "qgemm_b8"),
         ("rows.hip", [], "rows"), ("attn.hip", [], "attn"), ("lmhead.hip", [], "lmhead"),
         ("engine.cpp", [], "engine"), ("sched.cpp", [], "sched"), ("synth.cpp", [], "synth"),
         ("intfer_file.cpp", [], "intfer_file"), ("serve.cpp", [], "serve"),
         ("sample.cpp", [], "sample"), ("qgemm_f16.hip", [], "qgemm_f16"),
           ("qgemm_ga.hip", [], "qgemm_ga"), ("peak.hip", [], "peak")]

FLAGS = ["-O1", "-g", "-fPIC", "-std=c++17", "-fsanitize=address", "-fno-omit-frame-pointer",
         "-ffp-contract=off", "-Wno-unused-command-line-argument", "-w",
         f"-I{HERE}", f"-I{SRC}", f"-I{ROOT / 'include'}"]

_EXTERN_SHARED = re.compile(r"extern\s+__shared__\s+([\w:]+)\s+(\w+)\s*\[\s*\]\s*;")


def asan_runtime() -> str:
    hits = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
    if not hits:
        raise RuntimeError("clang ASan runtime not found")
    return hits[0]


def _transform() -> None:
    SRC.mkdir(parents=True, exist_ok=True)
    for p in CSRC.iterdir():
        if p.suffix not in (".hip", ".cpp", ".h"):
            continue
        t = p.read_text()
        t = _EXTERN_SHARED.sub(lambda m: f"{m.group(1)}* {m.group(2)} = "
                                         f"reinterpret_cast<{m.group(1)}*>(::emu::dyn_shared());", t)
        t = t.replace('"+v"', '"+x"')
        dst = SRC / p.name
        if not dst.exists() or dst.read_text() != t:
            dst.write_text(t)


def _deps(path: Path) -> list[Path]:
    return [path, HERE / "hip" / "hip_runtime.h", *SRC.glob("*.h"), ROOT / "include" / "intfer_amd.h"]


def _compile(item):
    src, defs, name = item
    path = HERE / "emu.cpp" if src == "emu.cpp" else SRC / src
    obj = BUILD / f"{name}.o"
    if obj.exists() and all(obj.stat().st_mtime >= d.stat().st_mtime for d in _deps(path)):
        return obj
    cmd = [CLANG, *FLAGS, *defs, "-x", "c++", "-c", str(path), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"emu compile failed for {src}:\n{r.stderr[-5000:]}")
    return obj


def build(jobs: int = 8) -> Path:
    _transform()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, UNITS + [("emu.cpp", [], "emu")]))
    rt = Path(asan_runtime()).parent
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [CLANG, "-shared", "-fsanitize=address", "-shared-libasan", f"-Wl,-rpath,{rt}", *map(str, objs),
           "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"emu link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)  # a new inode: processes still running the old one are unaffected
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
