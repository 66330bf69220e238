"""Host-side copy checker of the grouped GEMM (runs on the CPU).

Builds tests/native/gemm_copy_check (the library's host code with every optional path switched
on, linked with host versions of the GEMM launches that replay each kernel's copy schedule) and
runs its scenarios: the grouped GEMM C-ABI (bf16 / MXFP8, EIO / EOI weights, decode-shaped groups,
more groups than the LDS tile prefix holds), the MegaMoE forward (both precisions and layouts, the
numerics options) and the expert backward, on the 4-wave and decode kernels and (pp_* scenarios) on
the default 8-wave kernel of gemm_pp.hip (*_skinny: with its 384 x 128 tile switched on, MX and bf16; every call's launches must take each
group once). For every copy of every work item, wave and lane the
checker verifies the global source (inside a live allocation; for the 4-wave kernels also equal to
the element the fragment reads expect), the LDS destination slot and the slot coverage, and for the
4-wave kernels the vmcnt waits and the ring-slot reuse; the emu_* scenarios also run the kernels'
fragment reads, MFMAs and (8-wave) epilogues through an emulation of the lane-crossing instructions
and compare the results with a reference GEMM, and the 8-wave MXFP8 SwiGLU epilogue with the fp32
one followed by the MX quantisation; for the 4-wave and decode kernels they also run the text of the
epilogue (gemm_epilogue.inc, one host thread per kernel thread) on the emulated accumulators and compare
its stores with the reference GEMM and its fused MX requant byte for byte with an independent
quantiser; the mut_pp_* and mut_epi_* scenarios switch on deliberate faults of the replay and pass when
the checks report them. Decode-shaped forwards run the one-launch decode
prologue's code under a host emulation of its workgroup (prep_sim.inc) and compare its dispatch and
tile plan with the checker's own. See tests/native/gemm_copy_check.cpp, pp_sim.inc and prep_sim.inc.
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from tests.native import build_check


def _toolchain():
    return shutil.which("objcopy") and shutil.which("nm") and (build_check._rocm() / "bin" / "hipcc").exists()


@pytest.fixture(scope="module")
def checker():
    if not _toolchain():
        pytest.skip("hipcc / binutils not available")
    return build_check.build()


SCENARIOS = [
    "gemm_bf16_eio", "gemm_bf16_eoi", "gemm_bf16_eio_narrow", "gemm_bf16_eoi_narrow", "gemm_mx_eio", "gemm_mx_eoi",
    "gemm_mx_eoi_long_k", "gemm_mx_eio_long_k", "gemm_bf16_eio_decode", "gemm_bf16_eoi_decode", "gemm_mx_eio_decode",
    "gemm_mx_eoi_decode", "gemm_bf16_eio_decode_big", "gemm_bf16_eoi_decode_big", "gemm_mx_eio_decode_big",
    "moe_bf16_eio_decode_big", "moe_mx_eio_decode_big", "moe_bf16_gu_decode_big", "moe_mx_gu_decode_big",
    "moe_mx_decode_halves", "moe_mx_gu_decode_halves", "moe_bf16_decode_halves", "moe_bf16_gu_decode_halves",
    "moe_mx_eoi_decode_halves", "emu_bf16_eio", "emu_bf16_eoi", "emu_mx_eio", "emu_mx_eoi", "emu_bf16_eio_decode",
    "emu_bf16_eoi_decode", "emu_mx_eio_decode", "emu_mx_eoi_decode", "emu_moe_mx_decode_halves",
    "emu_moe_bf16_decode_halves", "emu_moe_mx_gu_decode_halves", "emu_wgrad_bf16", "emu_wgrad_mx",
    "pp_gemm_bf16_eio", "pp_gemm_bf16_eoi", "pp_gemm_bf16_eio_narrow", "pp_gemm_bf16_many_items",
    "pp_gemm_bf16_noalloc", "pp_moe_bf16_eio_prefill", "pp_moe_bf16_eoi_prefill", "pp_moe_bf16_gu_prefill",
    "pp_moe_mx_eio_prefill", "pp_moe_mx_gu_prefill", "pp_moe_mx_gu_skewed", "pp_moe_bf16_gu_skewed",
    "pp_moe_mx_gu_decode_variant", "pp_moe_bf16_eio_decode_variant", "pp_gemm_bf16_decode_variant",
    "pp_bf16_kn_store", "pp_mx_swiglu_gu", "emu_pp_bf16_kn_store", "emu_pp_bf16_nk_store",
    "emu_pp_bf16_kn_store_256", "emu_pp_bf16_kn_swiglu", "emu_pp_bf16_kn_swiglu_gu", "emu_pp_bf16_nk_swiglu",
    "emu_pp_mx_store", "emu_pp_mx_swiglu", "emu_pp_mx_swiglu_gu", "emu_pp_mx_skinny_store",
    "emu_pp_mx_skinny_swiglu", "emu_pp_mx_skinny_swiglu_gu", "emu_pp_bf16_nk_skinny_store_320",
    "emu_pp_bf16_nk_skinny_swiglu_320", "emu_pp_bf16_nk_skinny_store_256", "emu_pp_bf16_nk_skinny_swiglu_256",
    "emu_pp_bf16_kn_skinny_store_320", "emu_pp_bf16_kn_skinny_swiglu_256", "emu_pp_bf16_kn_skinny_swiglu_gu_320",
    "pp_moe_bf16_gu_skinny", "pp_moe_bf16_eio_skinny", "pp_moe_bf16_eoi_skinny", "pp_moe_mx_eio_skinny",
    "pp_moe_mx_gu_skinny", "gate_skinny_off", "gate_decode_prep_off", "pp_moe_mx_gu_skinny_none",
    "pp_moe_mx_gu_skinny_skewed", "emu_moe_bf16_numerics_clamp", "emu_moe_bf16_numerics_after_silu",
    "emu_moe_bf16_probs_before_fc2", "mut_epi_exp", "mut_epi_rounding", "mut_epi_scale", "mut_pp_copy_offset",
    "mut_pp_copy_oob", "mut_pp_copy_skipped", "mut_pp_staging", "mut_pp_shuffle", "mut_pp_rounding",
    "gemm_bf16_many_groups", "gemm_bf16_noalloc", "moe_bf16_eio", "moe_bf16_eoi", "moe_bf16_eio_prefill",
    "moe_mx_eio", "moe_mx_eoi", "moe_mx_eoi_prefill", "moe_mx_eio_prefill", "moe_mx_gu_prefill", "moe_bf16_gu",
    "moe_bf16_numerics_clamp", "moe_bf16_numerics_after_silu", "moe_bf16_probs_before_fc2", "bwd_eio_f32",
    "bwd_eoi_bf16", "bwd_eio_bf16_prefill", "bwd_mx_f32", "bwd_mx_bf16_prefill"
]


def test_scenario_list_matches(checker):
    """Every scenario the checker knows is run here (and no name here is unknown to it)."""
    r = subprocess.run([str(checker), "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == SCENARIOS


def _run(checker, name):
    return subprocess.run([str(checker), name], capture_output=True, text=True, timeout=600)


@pytest.fixture(scope="module")
def runs(checker):
    """Scenario name -> its run. In a plain pytest process the scenarios run as concurrent checker
    processes (one per host CPU, at most 8) when the first of them is needed; under pytest-xdist each
    test runs its own, since the workers already run in parallel."""
    if os.environ.get("PYTEST_XDIST_WORKER"):
        return None
    workers = max(1, min(8, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        futures = {name: pool.submit(_run, checker, name) for name in SCENARIOS}
        return {name: f.result() for name, f in futures.items()}


@pytest.mark.parametrize("name", SCENARIOS)
def test_copy_schedule(checker, runs, name):
    r = runs[name] if runs is not None else _run(checker, name)
    assert r.returncode == 0, f"{r.stdout}\n{r.stderr}"
    assert f"{name}" in r.stdout and " ok " in r.stdout
    if name.startswith(("moe_", "emu_moe_")) and "decode" in name:
        # decode-shaped forwards take the one-launch prologue (its code under the host emulation)
        assert "preps=1" in r.stdout, r.stdout
