"""Read-bandwidth ceiling of one MI355X for loads issued from the CUs (measurement, not product).

``build()`` compiles ``read_ceiling.hip`` into ``libreadceiling.so`` beside it; ``sweep()`` times each
kernel configuration over a buffer far larger than the last-level caches with HIP events on torch's
current stream (the stream the kernels are launched on) and returns GB/s per configuration.
``python tests/native/read_ceiling.py [--json PATH]`` prints the table.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "read_ceiling.hip"
LIB = HERE / "libreadceiling.so"

# (family, grid per CU, unroll or KB per step, ring depth)
CONFIGS = [
    ("regs", 4, 4, 0), ("regs", 8, 4, 0), ("regs", 16, 4, 0), ("regs", 8, 8, 0), ("regs", 16, 8, 0),
    ("regs", 32, 2, 0), ("regs", 32, 4, 0),
    ("lds", 1, 4, 1), ("lds", 1, 4, 2), ("lds", 1, 4, 4), ("lds", 1, 8, 1), ("lds", 1, 8, 2),
    ("lds", 1, 2, 2), ("lds", 1, 2, 4), ("lds", 1, 2, 8), ("lds", 1, 1, 8),
]


def build() -> Path:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = [str(Path(rocm) / "bin" / "hipcc"), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", str(SRC), "-o", str(LIB) + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("hipcc failed for read_ceiling.hip")
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


def load():
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    lib.read_ceiling_regs.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]
    lib.read_ceiling_lds.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_void_p]
    lib.read_ceiling_lds_bytes.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    lib.read_ceiling_lds_bytes.restype = ctypes.c_int64
    return lib


def sweep(gib: float = 4.0, reps: int = 10, configs=CONFIGS):
    import torch
    lib = load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    nbytes = int(gib * (1 << 30))
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    sink = torch.zeros(cus * 32 * 256 * 16, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    out = []
    for fam, per_cu, u, d in configs:
        grid = cus * per_cu
        if fam == "regs":
            run = lambda: lib.read_ceiling_regs(buf.data_ptr(), nbytes, grid, u, sink.data_ptr(), st)
            moved = nbytes
            name = f"regs grid={per_cu}x{cus} wg=256 unroll={u}"
        else:
            run = lambda: lib.read_ceiling_lds(buf.data_ptr(), nbytes, grid, u, d, sink.data_ptr(), st)
            moved = lib.read_ceiling_lds_bytes(nbytes, grid, u)
            name = f"lds grid={per_cu}x{cus} wg=512 kb_per_wave_step={u} depth={d}"
        rc = run()
        if rc != 0:
            raise RuntimeError(f"{name}: rc {rc}")
        for _ in range(2):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out.append({"config": name, "bytes": moved, "ms": round(ms, 4), "GBps": round(moved / ms / 1e6, 1)})
        print(f"[read_ceiling] {name}: {moved / ms / 1e6:.1f} GB/s ({ms:.4f} ms)", flush=True)
    assert int(sink.count_nonzero()) == 0
    return out


if __name__ == "__main__":
    res = sweep()
    if len(sys.argv) > 2 and sys.argv[1] == "--json":
        Path(sys.argv[2]).write_text(json.dumps(res, indent=1))
