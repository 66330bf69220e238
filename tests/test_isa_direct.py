"""Compiled-code checks of the direct-weight and split-role grouped GEMMs (CPU only; see
tests/native/isa_check.py).

The kernels load weight fragments into registers with inline assembly that the compiler does not
track, so their correctness also depends on the compiler's register allocation; these tests read the
gfx950 assembly hipcc builds from gemm_direct.hip and check that no register is touched while a load
into it is in flight, and that the steady K loop neither spills nor drains the load ring.
"""
import shutil
from pathlib import Path

import pytest

from tests.native import isa_check

SYNTH = """
_Z26grouped_gemm_direct_kernelILb0ELi0EEv8GGParams:
  s_waitcnt vmcnt(0)
  global_load_dwordx4 v[0:3], v10, s[2:3]
  global_load_lds_dwordx4 v11, s[4:5]
.LBB0_1:
  s_waitcnt vmcnt(1)
  v_mfma_f32_32x32x16_bf16 a[0:15], v[20:23], v[0:3], a[0:15]
  {use}
  global_load_dwordx4 v[0:3], v10, s[2:3]
  global_load_lds_dwordx4 v11, s[4:5]
""" + "  v_mfma_f32_32x32x16_bf16 a[0:15], v[20:23], v[24:27], a[0:15]\n" * 16 + """
  s_cbranch_scc1 .LBB0_1
  s_waitcnt vmcnt(0)
  s_endpgm
"""


def _findings(text, tmp_path):
    p = Path(tmp_path) / "k.s"
    p.write_text(text)
    return isa_check.run(p)


def test_checker_accepts_a_clean_pipeline(tmp_path):
    assert _findings(SYNTH.format(use="v_add_u32_e32 v30, v31, v32"), tmp_path) == []


@pytest.mark.parametrize("use", ["v_mov_b32_e32 v30, v1", "v_add_u32_e32 v2, v31, v32"])
def test_checker_flags_a_register_of_an_in_flight_load(tmp_path, use):
    # after the loop's loads are issued again, v[0:3] is in flight until the next wait
    text = SYNTH.format(use="v_add_u32_e32 v30, v31, v32").replace(
        "  s_cbranch_scc1 .LBB0_1", f"  {use}\n  s_cbranch_scc1 .LBB0_1")
    assert any("in-flight" in f for f in _findings(text, tmp_path))


def test_checker_flags_spills_and_drains_in_the_loop(tmp_path):
    text = SYNTH.format(use="scratch_load_dword v40, off, off offset:8\n  s_waitcnt vmcnt(0)")
    found = _findings(text, tmp_path)
    assert any("spill" in f for f in found) and any("every load" in f for f in found)


def test_checker_flags_a_vector_base(tmp_path):
    text = SYNTH.format(use="v_add_u32_e32 v30, v31, v32").replace("global_load_dwordx4 v[0:3], v10, s[2:3]",
                                                                   "global_load_dwordx4 v[0:3], v10, v[12:13]")
    assert any("scalar base" in f for f in _findings(text, tmp_path))


SPLIT_SYNTH = """
_Z19grouped_gemm_kernelI5GGCfgILi256ELb1EEv8GGParams:
  s_waitcnt vmcnt(0)
.LBB0_1:
{first}
  s_barrier
""" + "  v_mfma_f32_32x32x16_bf16 a[0:15], v[20:23], v[24:27], a[0:15]\n" * 16 + """
  global_load_lds_dwordx4 v11, s[4:5]
  s_barrier
{second}
  s_cbranch_scc1 .LBB0_1
  s_endpgm
"""


def test_split_checker_flags_spills_only_in_steady_loops(tmp_path):
    p = Path(tmp_path) / "s.s"
    mfmas = "  v_mfma_f32_32x32x16_bf16 a[0:15], v[20:23], v[24:27], a[0:15]\n" * 16
    spill = "  scratch_load_dword v40, off, off offset:8"
    p.write_text(SPLIT_SYNTH.format(first=spill, second=mfmas))  # both barrier intervals compute
    assert any("spill" in f for f in isa_check.run_split(p))
    p.write_text(SPLIT_SYNTH.format(first="", second=mfmas))
    assert isa_check.run_split(p) == []
    # a per-item path: one barrier interval is the prologue's wait only, so the loop is not a steady K loop
    p.write_text(SPLIT_SYNTH.format(first=spill, second=""))
    assert isa_check.run_split(p) == ["no K loop found in the split-role kernels"]


@pytest.mark.skipif(not (isa_check.Path("/opt/rocm/bin/hipcc").exists() or shutil.which("hipcc")),
                    reason="hipcc not available")
def test_direct_kernels_compiled_code(tmp_path):
    asm = Path(tmp_path) / "gemm_direct.s"
    isa_check.compile_asm(asm)
    assert isa_check.run(asm) == []


@pytest.mark.skipif(not (isa_check.Path("/opt/rocm/bin/hipcc").exists() or shutil.which("hipcc")),
                    reason="hipcc not available")
def test_split_role_kernels_compiled_code(tmp_path):
    """The split-role kernels (gemm_split.hip, MXFP8 and bf16 on EIO weights): no spill traffic in their
    steady K loops (the compiler's waits for spill reloads would drain the copy ring) and scalar bases
    for the offset-form copies."""
    asm = Path(tmp_path) / "gemm_split.s"
    isa_check.compile_asm_of(isa_check.REPO / "hyper_multicore_amd" / "csrc" / "gemm_split.hip", asm)
    assert isa_check.run_split(asm) == []
