"""Checks of the compiled gfx950 code of the direct-weight grouped GEMM (test infrastructure, CPU only).

The direct-weight kernels (hyper_multicore_amd/csrc/gemm_direct.hip) load weight fragments into
registers with inline assembly, so the compiler does not know that those registers are written
asynchronously: correctness needs its register allocation to leave an in-flight register alone
until the kernel's own ``s_waitcnt vmcnt`` has retired the load. This module compiles the file to
AMD assembly (``hipcc --cuda-device-only -S``, the code built here) and checks, for every K loop
(the software-pipelined ring turns) of every kernel, from the prologue that fills the ring through
the steady loop (twice round) to the last turn:

* no instruction reads or writes a register while a load into it is in flight (vector-memory
  operations retire in order and stores count too; each ``s_waitcnt vmcnt(N)`` leaves the N
  youngest outstanding);
* every weight load takes its base from scalar registers (the scalar-base + vector-offset form);
* the steady loop holds no scratch (spill) traffic and no wait for all loads (``vmcnt(0)``), which
  would drain the ring.

    python tests/native/isa_check.py      # prints one line per K loop, exit status 1 on a finding
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
SRC = REPO / "hyper_multicore_amd" / "csrc" / "gemm_direct.hip"
KERNEL = re.compile(r"^(_Z\d+grouped_gemm_direct_kernel\w+):")
LOOP_BRANCH = re.compile(r"\s*s_(?:cbranch_\w+|branch)\s+(\.LBB\w+)")
REG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")
VMCNT = re.compile(r"s_waitcnt\b.*\bvmcnt\((\d+)(?:\s*\+\s*(\d+))?\)")


def compile_asm(out: Path) -> None:
    hipcc = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    cmd = [str(hipcc), "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{REPO / 'include'}", "--cuda-device-only", "-S", str(SRC), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{r.stderr}")


def _regs(text: str) -> set[int]:
    out: set[int] = set()
    for m in REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _instructions(lines):
    for x in lines:
        t = x.split(";")[0].strip()
        if t and not t.startswith(".") and not t.endswith(":"):
            yield t


def _kernels(asm: list[str]):
    starts = [(i, m.group(1)) for i, l in enumerate(asm) if (m := KERNEL.match(l))]
    for i, name in starts:
        end = next(j for j in range(i, len(asm)) if "s_endpgm" in asm[j])
        yield name, asm[i:end]


def _k_loops(body: list[str]):
    """(start, end) of the innermost backward-branch loops that hold MFMAs (the ring turns)."""
    labels = {l.split(":")[0]: i for i, l in enumerate(body) if l.startswith(".LBB")}
    loops = []
    for i, l in enumerate(body):
        m = LOOP_BRANCH.match(l)
        if m and m.group(1) in labels and labels[m.group(1)] < i:
            a = labels[m.group(1)]
            if sum("v_mfma" in x for x in body[a:i]) >= 16:
                loops.append((a, i))
    return [(a, b) for a, b in loops if not any(a < a2 and b2 < b for a2, b2 in loops)]


def check_loop(body: list[str], a: int, b: int) -> list[str]:
    """Findings for the K loop body[a:b] with its prologue and last turn."""
    findings = []
    pre = body[max(0, a - 4000):a]
    drains = [j for j, x in enumerate(pre) if (m := VMCNT.search(x)) and int(m.group(1)) == 0]
    pre = pre[drains[-1] + 1:] if drains else pre
    loop = body[a:b]
    tail = []
    for x in body[b + 1:]:
        tail.append(x)
        m = VMCNT.search(x)
        if (m and int(m.group(1)) == 0) or "s_endpgm" in x:
            break
    for t in _instructions(loop):
        if t.startswith("scratch_"):
            findings.append(f"spill traffic in the steady loop: {t}")
        m = VMCNT.search(t)
        if m and int(m.group(1)) == 0:
            findings.append(f"wait for every load in the steady loop: {t}")
    outstanding: list[set[int]] = []
    for phase, seg in (("prologue", pre), ("loop", loop), ("loop", loop), ("last turn", tail)):
        for t in _instructions(seg):
            m = VMCNT.search(t)
            if m:
                n = int(m.group(1)) + int(m.group(2) or 0)
                del outstanding[:max(0, len(outstanding) - n)]
                continue
            op = t.split()[0]
            busy = set().union(*outstanding) if outstanding else set()
            if _regs(t) & busy:
                findings.append(f"{phase}: register of an in-flight load used: {t}")
            if op == "global_load_dwordx4":
                parts = [p.strip() for p in t[len(op):].split(",")]
                if len(parts) < 3 or not parts[2].startswith("s["):
                    findings.append(f"{phase}: weight load without a scalar base: {t}")
                outstanding.append(_regs(parts[0]))
            elif op.startswith(("global_load", "buffer_load", "scratch_load")):
                outstanding.append(_regs(t[len(op):].split(",")[0]) if "lds" not in op else set())
            elif op.startswith(("global_store", "buffer_store", "scratch_store", "global_atomic", "buffer_atomic")):
                outstanding.append(set())  # stores count in vmcnt on gfx9 as well
    return findings


def run(asm_path: Path | None = None) -> list[str]:
    """All findings (empty: the compiled code is as the pipeline needs); prints a line per loop."""
    tmp = None
    if asm_path is None:
        tmp = tempfile.TemporaryDirectory()
        asm_path = Path(tmp.name) / "gemm_direct.s"
        compile_asm(asm_path)
    asm = asm_path.read_text().split("\n")
    findings = []
    loops = 0
    for name, body in _kernels(asm):
        for a, b in _k_loops(body):
            f = check_loop(body, a, b)
            loops += 1
            print(f"{name}: K loop of {sum('v_mfma' in x for x in body[a:b])} MFMAs: {len(f)} findings")
            findings += [f"{name}: {x}" for x in f]
    if loops == 0:
        findings.append("no K loop found in the direct-weight kernels")
    if tmp is not None:
        tmp.cleanup()
    return findings


SPLIT_KERNEL = re.compile(r"^(_Z\d+grouped_gemm_kernelI5GGCfgI\w*Lb1EE\w*):")  # GGCfg<..., SPLIT = true>


def compile_asm_of(src: Path, out: Path) -> None:
    hipcc = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    cmd = [str(hipcc), "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{REPO / 'include'}", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{r.stderr}")


def _steady(ins: list[str]) -> bool:
    """True for a steady K loop: every interval between two of its workgroup barriers (taken
    cyclically, the loop repeats) holds MFMAs. The compiler also makes innermost loops of the
    persistent item loop for items of a stage or two, whose K work is the ring prologue and one step
    inlined: those have a barrier interval without MFMAs (the prologue's wait) and run once per item."""
    bars = [k for k, t in enumerate(ins) if t.startswith("s_barrier")]
    if not bars:
        return False
    cuts = bars + [bars[0] + len(ins)]
    cyc = ins + ins
    return all(any("v_mfma" in t for t in cyc[cuts[j]:cuts[j + 1]]) for j in range(len(bars)))


def run_split(asm_path: Path | None = None) -> list[str]:
    """Findings for the split-role kernels of gemm_split.hip: their steady K loops must hold no spill
    traffic, and their scalar-base copies must take the base from scalar registers."""
    tmp = None
    if asm_path is None:
        tmp = tempfile.TemporaryDirectory()
        asm_path = Path(tmp.name) / "gemm_split.s"
        compile_asm_of(REPO / "hyper_multicore_amd" / "csrc" / "gemm_split.hip", asm_path)
    asm = asm_path.read_text().split("\n")
    findings, loops = [], 0
    starts = [(i, m.group(1)) for i, l in enumerate(asm) if (m := SPLIT_KERNEL.match(l))]
    for i, name in starts:
        end = next(j for j in range(i, len(asm)) if "s_endpgm" in asm[j])
        body = asm[i:end]
        for t in _instructions(body):
            if t.startswith("global_load_lds_dwordx4"):
                parts = [p.strip() for p in t[len("global_load_lds_dwordx4"):].split(",")]
                if len(parts) < 2 or not (parts[1] == "off" or parts[1].startswith("s[")):
                    findings.append(f"{name}: copy without a scalar base: {t}")
        for a, b in _k_loops(body):
            ins = list(_instructions(body[a:b + 1]))
            if not _steady(ins):
                continue  # a per-item path (prologue and one step inside the persistent item loop)
            loops += 1
            spills = [t for t in ins if t.startswith("scratch_")]
            if spills:
                findings.append(f"{name}: {len(spills)} spill instructions in a K loop, e.g. {spills[0]}")
    if loops == 0:
        findings.append("no K loop found in the split-role kernels")
    if tmp is not None:
        tmp.cleanup()
    return findings


if __name__ == "__main__":
    found = run(Path(sys.argv[1]) if len(sys.argv) > 1 else None)
    for x in found[:40]:
        print(x)
    sys.exit(1 if found else 0)
