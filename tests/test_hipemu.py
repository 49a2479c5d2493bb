"""CPU bounds checking of the gfx950 kernels (no GPU needed).

The unmodified library sources are compiled for the host against a HIP
emulation (tests/hipemu: one fiber per GPU thread, lockstep exchange for
cross-lane operations and MFMA, __syncthreads as a block rendezvous) with
AddressSanitizer, and driven through the same C-ABI calls as the GPU tests on
small inputs.  Any out-of-bounds global/LDS/stack access, barrier mismatch or
divergent cross-lane operation aborts the run; results are also checked
against the CPU oracle.  The emulated library is only ever loaded here.
"""
import os
import shutil

import pytest

from tests.hipemu import build as eb
from tests.hipemu import runner


@pytest.fixture(scope="module")
def emu_lib():
    if not shutil.which(eb.CLANG):
        pytest.skip("host clang++ not available")
    try:
        eb.asan_runtime()
        eb.build()
    except Exception as e:  # toolchain problem, not a kernel finding
        pytest.skip(f"host emulation build unavailable: {e}")
    if runner.run_scenarios(["noop"], timeout=300) != 0:
        pytest.skip("ASan-preloaded child process cannot start here")
    return eb.LIB


# every scenario, longest first: the pool runs them side by side and each test
# waits for its own
ORDER = ["gemm_stream", "gemm_stream_rows", "gemm_full", "forward_fused_qk", "prefix_copy", "gemm_small",
         "forward_gated", "noalloc_limits", "gemm_grouped", "gemm_f16", "gemm_ga", "attention_ragged_g5",
         "forward_gqa5", "attention_ragged", "smoke", "act_quant", "intfer_load"]


@pytest.fixture(scope="module")
def emu_runs(emu_lib):
    pool = runner.ScenarioPool(ORDER, jobs=max(1, min(6, (os.cpu_count() or 2) - 2)))
    yield pool
    pool.close()


def test_small_model_forward_in_bounds(emu_runs):
    assert emu_runs.result(["smoke", "act_quant"], timeout=1800) == 0


def test_ragged_attention_in_bounds(emu_runs):
    assert emu_runs.result(["attention_ragged"], timeout=1800) == 0


def test_every_gemm_launch_shape_in_bounds(emu_runs):
    assert emu_runs.result(["gemm_small", "gemm_full", "gemm_stream", "gemm_stream_rows", "gemm_grouped",
                            "gemm_f16", "gemm_ga"], timeout=1800) == 0


def test_intfer_load_and_parser_in_bounds(emu_runs):
    assert emu_runs.result(["intfer_load"], timeout=1800) == 0


def test_gqa_group5_shapes_in_bounds(emu_runs):
    assert emu_runs.result(["attention_ragged_g5", "forward_gqa5"], timeout=1800) == 0


def test_noalloc_attention_at_its_limits_in_bounds(emu_runs):
    assert emu_runs.result(["noalloc_limits"], timeout=1800) == 0


def test_prefix_copy_and_cache_in_bounds(emu_runs):
    assert emu_runs.result(["prefix_copy"], timeout=1800) == 0


def test_fused_qk_epilogue_in_bounds_and_bit_identical(emu_runs):
    assert emu_runs.result(["forward_fused_qk"], timeout=1800) == 0


def test_attention_output_gate_in_bounds(emu_runs):
    assert emu_runs.result(["forward_gated"], timeout=1800) == 0
