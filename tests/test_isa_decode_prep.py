"""Compiled code of the one-launch decode prologue (CPU only).

dispatch.hip is compiled for gfx950 to AMD assembly (the code built here). decode_prep_kernel must
use no scratch memory, fit its LDS (the per-wave histogram rows, the tile counts and the scan
values) in one workgroup's share, take its histogram with LDS atomics only (no global atomics: the
result must not depend on scheduling), and copy the token blocks with 16-byte loads and stores.
"""
import os
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "hyper_multicore_amd" / "csrc"
HIPCC = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not HIPCC.exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "dispatch.s"
    cmd = [str(HIPCC), "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{REPO / 'include'}",
           str(CSRC / "dispatch.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def _kernel(asm, key):
    bodies, meta = {}, {}
    for m in re.finditer(r"^(_Z\w*" + key + r"\w*):", asm, re.M):
        end = asm.index(".Lfunc_end", m.end())
        lines = [l.split(";")[0].strip() for l in asm[m.end():end].splitlines()]
        bodies[m.group(1)] = [l for l in lines if l]
    md = asm[asm.index("amdhsa.kernels:"):]
    for block in re.split(r"\n  - ", md)[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        if name and key in name.group(1):
            get = lambda k: int(re.search(rf"\.{k}:\s+(\d+)", block).group(1))
            meta[name.group(1)] = {"vgpr": get("vgpr_count"), "private": get("private_segment_fixed_size"),
                                   "lds": get("group_segment_fixed_size")}
    return bodies, meta


def test_decode_prep_kernel_compiled_code(asm):
    bodies, meta = _kernel(asm, "decode_prep_kernel")
    assert len(bodies) == 2 and set(bodies) == set(meta)  # int32 and int64 ids
    for name, lines in bodies.items():
        m = meta[name]
        assert m["private"] == 0, (name, m)
        assert 16 * 1024 < m["lds"] <= 64 * 1024, (name, m)
        assert m["vgpr"] <= 128, (name, m)
        assert any(l.startswith("ds_add") for l in lines), name  # the LDS histogram
        assert not any(l.startswith("global_atomic") for l in lines), name
        assert any(l.startswith("global_load_dwordx4") for l in lines), name  # token blocks, 16 bytes
        assert any(l.startswith("global_store_dwordx4") for l in lines), name
