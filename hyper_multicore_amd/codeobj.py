"""Digests of the gfx950 kernels inside this package's own built library (measurement bookkeeping).

The committed counter records (profiles/traffic_*.json) hold the HBM bytes rocprofv3 counted for
one kernel. A record stays valid only while that kernel's machine code is unchanged, so each record
carries the kernel's symbol and ``code_digest``: a SHA-256 over the kernel's code bytes and its kernel
descriptor (the descriptor's code-entry offset, which moves when other kernels change size, left
out). The kernels branch only within themselves and load no data relative to the program counter,
so the bytes do not depend on where the linker put the kernel.

The library's device code is read from its ``.hip_fatbin`` section: clang offload bundles, one per
translation unit, whose gfx950 entries are ELF code objects. Only libraries built here are read.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import struct
import subprocess

_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
_TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _sections(elf: bytes) -> list[tuple[str, int, int, int, int, int]]:
    """(name, type, addr, offset, size, link) of every section of a little-endian ELF64 image."""
    if elf[:4] != b"\x7fELF" or elf[4] != 2 or elf[5] != 1:
        raise ValueError("not a little-endian ELF64 image")
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    raw = []
    for i in range(shnum):
        name, typ, _flags, addr, off, size, link = struct.unpack_from("<IIQQQQI", elf, shoff + i * shentsize)
        raw.append((name, typ, addr, off, size, link))
    stroff, strsize = raw[shstrndx][3], raw[shstrndx][4]
    names = elf[stroff:stroff + strsize]
    out = []
    for name, typ, addr, off, size, link in raw:
        end = names.index(b"\0", name)
        out.append((names[name:end].decode(), typ, addr, off, size, link))
    return out


def _symbols(elf: bytes) -> dict[str, tuple[int, int, int]]:
    """name -> (value, size, section index) from .symtab."""
    secs = _sections(elf)
    syms = {}
    for name, typ, _addr, off, size, link in secs:
        if typ != 2:  # SHT_SYMTAB
            continue
        stroff = secs[link][3]
        for i in range(size // 24):
            st_name, _info, _other, shndx, value, ssize = struct.unpack_from("<IBBHQQ", elf, off + i * 24)
            if st_name == 0:
                continue
            end = elf.index(b"\0", stroff + st_name)
            syms[elf[stroff + st_name:end].decode()] = (value, ssize, shndx)
    return syms


def code_objects(lib_path: str) -> list[bytes]:
    """The gfx950 code objects in a shared library's .hip_fatbin section."""
    with open(lib_path, "rb") as f:
        so = f.read()
    fat = [s for s in _sections(so) if s[0] == ".hip_fatbin"]
    if not fat:
        raise ValueError(f"{lib_path}: no .hip_fatbin section")
    _, _, _, off, size, _ = fat[0]
    blob = so[off:off + size]
    objs, pos = [], 0
    while True:
        i = blob.find(_BUNDLE_MAGIC, pos)
        if i < 0:
            break
        count, = struct.unpack_from("<Q", blob, i + len(_BUNDLE_MAGIC))
        o = i + len(_BUNDLE_MAGIC) + 8
        for _ in range(count):
            eoff, esize, idlen = struct.unpack_from("<QQQ", blob, o)
            o += 24
            tid = blob[o:o + idlen].decode()
            o += idlen
            if tid == _TARGET and esize:
                objs.append(blob[i + eoff:i + eoff + esize])
        pos = i + len(_BUNDLE_MAGIC)
    return objs


def _bytes_of(elf: bytes, secs, value: int, size: int, shndx: int) -> bytes:
    _, _, addr, off, _, _ = secs[shndx]
    start = off + (value - addr)
    return elf[start:start + size]


def kernel_digests(lib_path: str) -> dict[str, str]:
    """Mangled kernel symbol -> code digest (16 hex digits) for every gfx950 kernel of the library."""
    out = {}
    for elf in code_objects(lib_path):
        secs = _sections(elf)
        syms = _symbols(elf)
        for name, (value, size, shndx) in syms.items():
            kd = syms.get(name + ".kd")
            if kd is None or size == 0:
                continue
            h = hashlib.sha256()
            h.update(_bytes_of(elf, secs, value, size, shndx))
            desc = _bytes_of(elf, secs, *kd)
            h.update(desc[:16] + desc[24:])  # without kernel_code_entry_byte_offset
            out[name] = h.hexdigest()[:16]
    return out


def demangle(names: list[str]) -> list[str]:
    """C++ demangling through llvm-cxxfilt (ROCm) or c++filt; the names unchanged when neither exists."""
    tool = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "llvm-cxxfilt")
    if not os.path.exists(tool):
        tool = shutil.which("c++filt")
    if tool is None:
        return list(names)
    r = subprocess.run([tool], input="\n".join(names) + "\n", capture_output=True, text=True, check=True)
    return r.stdout.splitlines()[:len(names)]


def find_kernel(lib_path: str, demangled: str) -> tuple[str, str] | None:
    """(mangled symbol, code digest) of the kernel whose demangled name is ``demangled``."""
    dig = kernel_digests(lib_path)
    names = sorted(dig)
    for mangled, plain in zip(names, demangle(names)):
        if plain == demangled:
            return mangled, dig[mangled]
    return None
