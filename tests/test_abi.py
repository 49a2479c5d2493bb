"""The C-ABI boundary without a GPU: the library loads, exports every function
the public header declares, the ctypes table binds exactly those, and the
host-side pieces (synthetic model, A-tile layout helpers) behave."""
import ctypes as C
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

import intfer_amd as ia
from intfer_amd import _abi

ROOT = Path(__file__).resolve().parents[1]


def test_library_exports_every_header_function():
    L = ia.lib()
    names = _abi.header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in intfer_amd.h but not exported: {missing}"


def test_ctypes_table_matches_header():
    names = set(_abi.header_functions())
    bound = set(_abi._PROTOS)
    assert bound == names, (sorted(names - bound), sorted(bound - names))


def test_default_cfg_is_the_headline_model():
    c = ia.default_cfg()
    assert (c.hidden, c.layers, c.n_heads, c.n_kv, c.head_dim, c.inter, c.vocab) == \
        (1024, 28, 16, 8, 128, 3072, 151936)
    assert c.qk_norm == 1 and c.rotate == 1 and c.group_size == 128
    assert abs(c.rms_eps - 1e-6) < 1e-12 and c.rope_theta == 1e6


def test_synth_model_is_deterministic():
    cfg = ia.default_cfg(layers=2, vocab=512, hidden=256, inter=384, n_heads=4, n_kv=2)
    a, b = ia.SynthModel(cfg, seed=3, bits=2), ia.SynthModel(cfg, seed=3, bits=2)
    c = ia.SynthModel(cfg, seed=4, bits=2)
    try:
        ea, eb, ec = a.embed(), b.embed(), c.embed()
        assert np.array_equal(ea, eb) and not np.array_equal(ea, ec)
        assert abs(float(ea.std()) - 0.02) < 2e-3
        la, lb = a.layer(1).down, b.layer(1).down
        nbytes = la.N * la.K * la.bits // 8
        ca = np.ctypeslib.as_array(C.cast(la.codes, C.POINTER(C.c_uint8)), shape=(nbytes,))
        cb = np.ctypeslib.as_array(C.cast(lb.codes, C.POINTER(C.c_uint8)), shape=(nbytes,))
        assert np.array_equal(ca, cb)
        ng = la.K // la.group
        sa = np.ctypeslib.as_array(C.cast(la.scale, C.POINTER(C.c_uint16)), shape=(la.N * ng,))
        sb = np.ctypeslib.as_array(C.cast(lb.scale, C.POINTER(C.c_uint16)), shape=(la.N * ng,))
        assert np.array_equal(sa, sb)
    finally:
        for m in (a, b, c):
            m.close()


@pytest.mark.parametrize("M,K", [(1, 64), (16, 128), (37, 1024), (130, 3072)])
def test_atile_round_trip(M, K):
    rng = np.random.default_rng(M * K)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    t = ia.atile(q)
    assert t.size == (M + 15) // 16 * 16 * K
    assert np.array_equal(ia.untile(t, M, K), q)


def test_atile_matches_header_macro():
    """The Python helper and IFR_ATILE_OFF of the C header agree (a small C
    program including the header prints the offsets)."""
    src = r"""
    #include <stdio.h>
    #include "intfer_amd.h"
    int main(void) {
      const int K = 192;
      for (int m = 0; m < 40; m += 3)
        for (int k = 0; k < K; k += 5) printf("%zu\n", (size_t)IFR_ATILE_OFF(m, k, K));
      return 0;
    }
    """
    with tempfile.TemporaryDirectory() as d:
        c, exe = Path(d) / "t.cpp", Path(d) / "t"
        c.write_text(src)
        subprocess.run(["g++", "-std=c++17", f"-I{ROOT / 'include'}", str(c), "-o", str(exe)], check=True)
        offs = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                               check=True).stdout.split()]
    # place a single nonzero at (m, k) and find where the helper puts it
    M, K = 40, 192
    for m in range(0, 40, 3):
        for k in range(0, K, 5):
            q = np.zeros((M, K), dtype=np.int8)
            q[m, k] = 1
            t = ia.atile(q)
            assert int(np.flatnonzero(t)[0]) == offs.pop(0), (m, k)
    assert not offs


def test_errors_without_device_are_reported():
    """Entry points reject null arguments with IFR_EINVAL and a message."""
    L = ia.lib()
    rc = L.ifr_quant_gemm(None, None, None, None, None, 1, None, None)
    assert rc == ia.IFR_EINVAL
    assert L.ifr_last_error()
