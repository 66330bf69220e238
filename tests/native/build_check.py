"""Build the host-side grouped-GEMM copy checker (test infrastructure, CPU only).

The library sources are compiled for the host only (``--cuda-host-only``) with every optional path
switched on, AddressSanitizer and UndefinedBehaviorSanitizer, the internal enqueue functions the
checker replaces are made weak, and everything is linked with ``gemm_copy_check.cpp`` and no HIP
runtime. Output goes to ``tests/native/_build`` (git-ignored); a build is reused while no input
changed.

    python tests/native/build_check.py      # builds and prints the binary paths

``build_prep()`` builds ``prep_check``: the one-launch decode prologue (decode_prep.h) under the host
emulation of ``prep_sim.inc``, with the same sanitizers.
"""
from __future__ import annotations

import fcntl
import hashlib
import os
import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
CSRC = REPO / "hyper_multicore_amd" / "csrc"
OUT = HERE / "_build"
LIB_SOURCES = ["api.hip", "backward.hip", "dispatch.hip", "quant.hip", "gemm.hip", "gemm_pp.hip"]
# internal functions defined by the checker instead (made weak in the library objects)
REPLACED = {
    "gemm.hip": ["mi355_grouped_gemm", "mi355_plan_tiles", "mi355_plan_row_blocks"],
    "dispatch.hip": ["mi355_dispatch_enqueue", "mi355_dispatch_plan_enqueue", "mi355_permute_rows_enqueue", "mi355_unpermute_enqueue",
                     "mi355_zero_enqueue", "mi355_decode_prep_enqueue"],
    "quant.hip": ["mi355_mx_quant_rows", "mi355_mx_quant_grouped"],
    "gemm_pp.hip": ["mi355_grouped_gemm_pp"],
}
# internal functions the checker wraps: linked under the name with the suffix `_lib`
RENAMED = {"gemm_pp.hip": ["mi355_gg_pp_usable"]}
# AddressSanitizer and UndefinedBehaviorSanitizer (any report ends the run), except the check on
# pointer arithmetic from a null base: the copy plans of waves that copy no scales hold a null scale
# pointer, and the kernels form (never dereference) its stage addresses for the predicated-off copies
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize=pointer-overflow", "-fno-sanitize-recover=undefined"]
FLAGS = ["-x", "hip", "--cuda-host-only", "-O1", "-g", "-std=c++17", *SANITIZE,
         "-fno-omit-frame-pointer", "-Wno-unused-result", "-Wno-unused-variable",
         f"-I{REPO / 'include'}"]


def _rocm() -> Path:
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _inputs() -> list[Path]:
    files = [CSRC / f for f in LIB_SOURCES] + sorted(CSRC.glob("*.h")) + sorted(CSRC.glob("*.inc"))
    return files + [REPO / "include" / "mi355moe.h", HERE / "gemm_copy_check.cpp", HERE / "pp_sim.inc", HERE / "prep_sim.inc",
                     Path(__file__)]


def _digest() -> str:
    h = hashlib.sha256()
    for f in _inputs():
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r.stdout


def build() -> Path:
    """Build the checker once per source digest; concurrent callers (pytest-xdist workers) wait on a
    file lock instead of building the same objects at the same time."""
    OUT.mkdir(parents=True, exist_ok=True)
    with open(OUT / ".lock", "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        return _build_locked()


def _build_locked() -> Path:
    exe = OUT / "gemm_copy_check"
    stamp = OUT / "stamp"
    digest = _digest()
    if exe.exists() and stamp.exists() and stamp.read_text() == digest:
        return exe
    hipcc = str(_rocm() / "bin" / "hipcc")
    objs = []
    for src in LIB_SOURCES:
        obj = OUT / (Path(src).stem + ".o")
        _run([hipcc, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        names = REPLACED.get(src, [])
        if names:
            syms = _run(["nm", str(obj)]).split()
            weak = [s for s in syms if any(re.fullmatch(rf"_Z\d+{n}\w*", s) for n in names)]
            if len(weak) < len(names):
                raise RuntimeError(f"{src}: expected symbols {names}, found {weak}")
            _run(["objcopy", *[f"--weaken-symbol={s}" for s in weak], str(obj)])
        for n in RENAMED.get(src, []):
            syms = _run(["nm", str(obj)]).split()
            found = [s for s in syms if re.fullmatch(rf"_Z{len(n)}{n}\w*", s)]
            if len(found) != 1:
                raise RuntimeError(f"{src}: expected one symbol {n}, found {found}")
            new = found[0].replace(f"_Z{len(n)}{n}", f"_Z{len(n) + 4}{n}_lib", 1)
            _run(["objcopy", f"--redefine-sym={found[0]}={new}", str(obj)])
        objs.append(obj)
    chk = OUT / "gemm_copy_check.o"
    _run([hipcc, *FLAGS, "-c", str(HERE / "gemm_copy_check.cpp"), "-o", str(chk)])
    objs.append(chk)
    # host-only objects refer to the (absent) device code images by name: define empty ones
    fat = set()
    for o in objs:
        fat.update(s for s in _run(["nm", "-u", str(o)]).split() if s.startswith("__hip_fatbin"))
    stub = OUT / "fatbin_stub.c"
    stub.write_text("".join(f"const char {s}[8] = {{0}};\n" for s in sorted(fat)))
    stub_o = OUT / "fatbin_stub.o"
    _run(["gcc", "-c", str(stub), "-o", str(stub_o)])
    clangxx = str(_rocm() / "llvm" / "bin" / "clang++")
    _run([clangxx, *SANITIZE, "-pthread", *map(str, objs), str(stub_o), "-o", str(exe)])
    stamp.write_text(digest)
    return exe


PREP_INPUTS = [CSRC / "decode_prep.h", CSRC / "common.h", HERE / "prep_sim.inc", HERE / "prep_check.cpp"]


def build_prep() -> Path:
    """Build tests/native/_build/prep_check once per source digest (same lock as build())."""
    OUT.mkdir(parents=True, exist_ok=True)
    with open(OUT / ".lock", "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        exe = OUT / "prep_check"
        stamp = OUT / "prep_stamp"
        h = hashlib.sha256()
        for f in PREP_INPUTS + [Path(__file__)]:
            h.update(f.name.encode())
            h.update(f.read_bytes())
        digest = h.hexdigest()[:16]
        if exe.exists() and stamp.exists() and stamp.read_text() == digest:
            return exe
        hipcc = str(_rocm() / "bin" / "hipcc")
        obj = OUT / "prep_check.o"
        _run([hipcc, *FLAGS, "-c", str(HERE / "prep_check.cpp"), "-o", str(obj)])
        clangxx = str(_rocm() / "llvm" / "bin" / "clang++")
        _run([clangxx, *SANITIZE, "-pthread", str(obj), "-o", str(exe)])
        stamp.write_text(digest)
        return exe


if __name__ == "__main__":
    print(build())
    print(build_prep())
    sys.exit(0)
