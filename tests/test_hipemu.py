"""CPU bounds checking of the gfx950 kernels (no GPU needed).

The unmodified library sources are compiled for the host against a HIP
emulation (tests/hipemu: one fiber per GPU thread, lockstep exchange for
cross-lane operations and MFMA, __syncthreads as a block rendezvous) with
AddressSanitizer, and driven through the same C-ABI calls as the GPU tests on
small inputs.  Any out-of-bounds global/LDS/stack access, barrier mismatch or
divergent cross-lane operation aborts the run; results are also checked
against the CPU oracle.  The emulated library is only ever loaded here.
"""
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


def test_small_model_forward_in_bounds(emu_lib):
    assert runner.run_scenarios(["smoke", "act_quant"], timeout=900) == 0


def test_ragged_attention_in_bounds(emu_lib):
    assert runner.run_scenarios(["attention_ragged"], timeout=900) == 0


def test_every_gemm_launch_shape_in_bounds(emu_lib):
    assert runner.run_scenarios(["gemm_small", "gemm_full", "gemm_stream", "gemm_stream_rows", "gemm_grouped",
                                 "gemm_f16", "gemm_ga"],
                                timeout=1800) == 0


def test_intfer_load_and_parser_in_bounds(emu_lib):
    assert runner.run_scenarios(["intfer_load"], timeout=600) == 0


def test_gqa_group5_shapes_in_bounds(emu_lib):
    assert runner.run_scenarios(["attention_ragged_g5", "forward_gqa5"], timeout=900) == 0


def test_noalloc_attention_at_its_limits_in_bounds(emu_lib):
    assert runner.run_scenarios(["noalloc_limits"], timeout=1200) == 0


def test_prefix_copy_and_cache_in_bounds(emu_lib):
    assert runner.run_scenarios(["prefix_copy"], timeout=900) == 0


def test_fused_qk_epilogue_in_bounds_and_bit_identical(emu_lib):
    assert runner.run_scenarios(["forward_fused_qk"], timeout=900) == 0


def test_attention_output_gate_in_bounds(emu_lib):
    assert runner.run_scenarios(["forward_gated"], timeout=900) == 0
