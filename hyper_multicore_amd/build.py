"""Build the gfx950 HIP library ``libmi355moe.so`` in-tree with hipcc.

The library is a plain C ABI (``include/mi355moe.h``); Python binds it with ctypes. The build
always recompiles (it is cheap) so that ``__graft_entry__.build()`` is a real build check.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
OUT_DIR = PACKAGE_DIR / "_lib"
LIB_NAME = "libmi355moe.so"
SOURCES = ["router.hip", "dispatch.hip", "gemm.hip", "gemm_wgrad.hip", "gemm_pp.hip", "quant.hip", "backward.hip", "api.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops are kept off for correctness on this fleet
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{REPO_DIR / 'include'}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed for {src.name}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link ``_lib/libmi355moe.so``; return its path."""
    OUT_DIR.mkdir(exist_ok=True)
    objs = [OUT_DIR / (Path(s).stem + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as pool:
        list(pool.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, lib)
    for o in objs:
        o.unlink(missing_ok=True)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True)
