"""Register budget of the default 8-wave grouped GEMM (CPU only).

gemm_pp.hip runs 8 waves per CU, two per SIMD, so each wave has 256 registers (VGPRs and AGPRs).
The kernels' design (gemm_pp_plan.h) relies on it: the MXFP8 kernels (256 x 256 and 384 x 128)
spill nothing, and the bf16
320-row kernels spill one 64-bit value outside the stage loops (a reload inside the loop would wait
for all outstanding copies). This test compiles gemm_pp.hip for gfx950 to AMD assembly (the code
built here) and checks, for every kernel, the register count, the spill size and that no scratch
access sits inside a loop (between a label and a backward branch to it).
"""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "hyper_multicore_amd" / "csrc"
HIPCC = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"


def _kernels(asm: str):
    """name -> (instruction lines, metadata dict) for every gg_pp_kernel in the assembly."""
    out = {}
    for m in re.finditer(r"^(_ZN\w*gg_pp_kernel\w*):", asm, re.M):
        name = m.group(1)
        end = asm.index(".Lfunc_end", m.end())
        body = [l.split(";")[0].strip() for l in asm[m.end():end].splitlines()]
        out[name] = [l for l in body if l]
    meta = {}
    kernels_md = asm[asm.index("amdhsa.kernels:"):]
    for block in re.split(r"\n  - ", kernels_md)[1:]:  # one metadata map per kernel
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name or "gg_pp_kernel" not in name.group(1):
            continue
        get = lambda k: int(re.search(rf"\.{k}:\s+(\d+)", block).group(1))
        meta[name.group(1)] = {"vgpr": get("vgpr_count"), "private": get("private_segment_fixed_size")}
    return out, meta


def _scratch_in_loops(lines):
    labels = {l[:-1]: i for i, l in enumerate(lines) if re.fullmatch(r"\.LBB\w+:", l)}
    found = []
    for i, l in enumerate(lines):
        m = re.match(r"s_(?:cbranch_\w+|branch)\s+(\.LBB\w+)", l)
        if m and m.group(1) in labels and labels[m.group(1)] < i:
            body = lines[labels[m.group(1)]:i]
            found += [x for x in body if x.startswith("scratch_")]
    return found


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not HIPCC.exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "gemm_pp.s"
    cmd = [str(HIPCC), "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{REPO / 'include'}",
           str(CSRC / "gemm_pp.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def test_pp_kernels_register_budget(asm):
    bodies, meta = _kernels(asm)
    assert len(bodies) >= 14 and set(bodies) == set(meta)
    assert any(re.search(r"ILb1ELb1ELi\d+ELb0ELi2E", n) for n in bodies)  # the 384 x 128 MX tile
    assert any(re.search(r"ILb0ELb0ELi\d+ELb0ELi[23]E", n) for n in bodies)  # the 384 x 128 bf16 tile
    for name, lines in bodies.items():
        # gg_pp_kernel<MX, B_KN, EPI, TALL, SEL>
        args = re.search(r"gg_pp_kernelILb(\d)ELb(\d)ELi(\d+)ELb(\d)ELi(\d)EEEv8GGParams", name)
        assert args, name
        mx, tall = args.group(1) == "1", args.group(4) == "1"  # SEL 2 / 3: the 384 x 128 tile
        m = meta[name]
        assert m["vgpr"] <= 256, (name, m)
        if mx or not tall:
            assert m["private"] == 0, (name, m)  # spill-free (the MX kernels, the 384 x 128 one included)
        else:
            assert m["private"] <= 16, (name, m)
        assert _scratch_in_loops(lines) == [], name
        assert any("global_load_lds_dwordx4" in l for l in lines)


def test_scratch_in_loop_detection():
    """The loop check finds a scratch access between a label and a backward branch to it, and only
    there."""
    lines = [".LBB0_1:", "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]", "scratch_load_dwordx2 v[8:9], off, off",
             "s_cbranch_scc1 .LBB0_1", "scratch_store_dwordx2 off, v[8:9], off", "s_branch .LBB0_2", ".LBB0_2:"]
    assert _scratch_in_loops(lines) == ["scratch_load_dwordx2 v[8:9], off, off"]
    assert _scratch_in_loops(lines[4:]) == []


def test_pp_kernels_have_stage_loops(asm):
    """Every kernel has backward branches (its stage loops), so the scratch check above inspects them."""
    bodies, _ = _kernels(asm)
    for name, lines in bodies.items():
        labels = {l[:-1]: i for i, l in enumerate(lines) if re.fullmatch(r"\.LBB\w+:", l)}
        back = [i for i, l in enumerate(lines)
                if (m := re.match(r"s_(?:cbranch_\w+|branch)\s+(\.LBB\w+)", l)) and labels.get(m.group(1), 1 << 30) < i]
        assert len(back) >= 2, name
