"""TEST INFRASTRUCTURE ONLY - compile the C oracle (router_ref.c) into oracle/_build/.

gcc with contraction and fast-math disabled, so the float operation order is the one written.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
LIB = BUILD_DIR / "librouter_ref.so"


def build() -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-shared", "-fPIC",
           str(ORACLE_DIR / "router_ref.c"), "-o", str(LIB), "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


def load() -> ctypes.CDLL:
    src = ORACLE_DIR / "router_ref.c"
    if not LIB.exists() or LIB.stat().st_mtime < src.stat().st_mtime:
        build()
    lib = ctypes.CDLL(str(LIB))
    lib.oracle_det_expf.restype = ctypes.c_float
    lib.oracle_det_expf.argtypes = [ctypes.c_float]
    lib.oracle_det_logf.restype = ctypes.c_float
    lib.oracle_det_logf.argtypes = [ctypes.c_float]
    vp = ctypes.c_void_p
    lib.oracle_route.restype = ctypes.c_int
    lib.oracle_route.argtypes = [vp, ctypes.c_int64, ctypes.c_int, vp, vp, vp, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_float, vp, vp, vp]
    lib.oracle_route_grad.restype = ctypes.c_int
    lib.oracle_route_grad.argtypes = [vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_float, ctypes.c_int, vp]
    return lib


if __name__ == "__main__":
    print(build())
