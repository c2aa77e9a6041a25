"""Resource usage of the compiled gfx950 kernels of liborthocache_hip.so.

The MI355X counterpart of the reference's print_kernel_metadata
(triton_kernels/fwht_fused_prototype.py:329-385, which reads Triton's
compiled-kernel metadata: shared memory, registers, spills).  Here every
kernel is compiled ahead of time, so the figures come from the AMDGPU
metadata note (NT_AMDGPU_METADATA, a msgpack map) of each gfx950 code
object bundled in the library's .hip_fatbin section: VGPRs, AGPRs, SGPRs,
LDS bytes per workgroup, scratch bytes per lane, and the VGPR / SGPR spill
counts.  Nothing is executed and no GPU is needed.

A kernel with scratch (private segment) bytes either spills registers to
memory or keeps a stack frame; the build keeps every kernel at zero
(tests/test_kernel_resources.py).
"""

from __future__ import annotations

import os
import shutil
import struct
import subprocess
from typing import Dict, List, Optional

_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
_NT_AMDGPU_METADATA = 32
_SHT_NOTE = 7


def library_path() -> str:
    """The in-tree library (orthocache_gpu/_lib/liborthocache_hip.so)."""
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "liborthocache_hip.so")


def _elf_section(data: bytes, name: bytes) -> Optional[bytes]:
    """Contents of the named section of a little-endian ELF64 file."""
    if data[:4] != b"\x7fELF" or data[4] != 2:
        raise ValueError("not an ELF64 file")
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    str_off, = struct.unpack_from("<Q", data, shoff + shstrndx * shentsize + 0x18)
    for i in range(shnum):
        sh = shoff + i * shentsize
        nm, = struct.unpack_from("<I", data, sh)
        end = data.index(b"\0", str_off + nm)
        if data[str_off + nm:end] == name:
            off, size = struct.unpack_from("<QQ", data, sh + 0x18)
            return data[off:off + size]
    return None


def _code_objects(fatbin: bytes, arch: str) -> List[bytes]:
    """The code objects for `arch` in a sequence of clang offload bundles."""
    out = []
    pos = fatbin.find(_BUNDLE_MAGIC)
    while pos >= 0:
        n, = struct.unpack_from("<Q", fatbin, pos + len(_BUNDLE_MAGIC))
        p = pos + len(_BUNDLE_MAGIC) + 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            triple = fatbin[p + 24:p + 24 + tlen].decode(errors="replace")
            p += 24 + tlen
            if size and triple.startswith("hip") and triple.endswith(arch):
                out.append(fatbin[pos + off:pos + off + size])
        pos = fatbin.find(_BUNDLE_MAGIC, pos + 1)
    return out


def _amdgpu_notes(elf: bytes) -> List[dict]:
    """The decoded NT_AMDGPU_METADATA notes of one code object."""
    import msgpack

    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
    notes = []
    for i in range(shnum):
        sh = shoff + i * shentsize
        typ, = struct.unpack_from("<I", elf, sh + 4)
        if typ != _SHT_NOTE:
            continue
        off, size = struct.unpack_from("<QQ", elf, sh + 0x18)
        p = off
        while p + 12 <= off + size:
            namesz, descsz, ntype = struct.unpack_from("<III", elf, p)
            p += 12
            owner = elf[p:p + namesz].rstrip(b"\0")
            p += (namesz + 3) & ~3
            desc = elf[p:p + descsz]
            p += (descsz + 3) & ~3
            if owner == b"AMDGPU" and ntype == _NT_AMDGPU_METADATA:
                notes.append(msgpack.unpackb(desc))
    return notes


def _demangle(names: List[str]) -> List[str]:
    tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
    if not tool:
        return names
    try:
        res = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True, timeout=30,
                             check=True)
    except (OSError, subprocess.SubprocessError):
        return names
    out = res.stdout.splitlines()
    return out if len(out) == len(names) else names


def kernel_metadata(path: Optional[str] = None, arch: str = "gfx950", demangle: bool = True) -> List[Dict]:
    """One dict per kernel of the library at `path` (default: the in-tree
    build): name (demangled when c++filt is present), symbol, vgpr,
    agpr, sgpr, lds_bytes, scratch_bytes (per lane), vgpr_spills,
    sgpr_spills, max_workgroup, wavefront."""
    path = path or library_path()
    with open(path, "rb") as f:
        lib = f.read()
    fat = _elf_section(lib, b".hip_fatbin")
    if fat is None:
        raise ValueError(f"{path} has no .hip_fatbin section")
    rows = []
    for co in _code_objects(fat, arch):
        for note in _amdgpu_notes(co):
            for k in note.get("amdhsa.kernels", []):
                rows.append({
                    "symbol": k[".name"],
                    "vgpr": k[".vgpr_count"],
                    "agpr": k.get(".agpr_count", 0),
                    "sgpr": k[".sgpr_count"],
                    "lds_bytes": k[".group_segment_fixed_size"],
                    "scratch_bytes": k[".private_segment_fixed_size"],
                    "vgpr_spills": k.get(".vgpr_spill_count", 0),
                    "sgpr_spills": k.get(".sgpr_spill_count", 0),
                    "max_workgroup": k[".max_flat_workgroup_size"],
                    "wavefront": k[".wavefront_size"],
                })
    names = [r["symbol"] for r in rows]
    for r, n in zip(rows, _demangle(names) if demangle else names):
        r["name"] = n
    return rows


def scratch_instructions(symbols: List[str], path: Optional[str] = None, arch: str = "gfx950") -> Dict[str, int]:
    """Scratch-memory instructions (scratch_load / scratch_store, gfx950's
    flat scratch) in the disassembly of each named kernel of the library, by
    llvm-objdump over the library's own code objects.  A kernel can carry a
    stack frame that no instruction touches (a spill slot the register
    allocator created and later emptied); this tells such frames from real
    scratch traffic."""
    import tempfile

    tool = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
    path = path or library_path()
    with open(path, "rb") as f:
        fat = _elf_section(f.read(), b".hip_fatbin")
    want = set(symbols)
    counts: Dict[str, int] = {}
    with tempfile.TemporaryDirectory() as tmp:
        for i, co in enumerate(_code_objects(fat, arch)):
            syms = [k[".name"] for note in _amdgpu_notes(co) for k in note.get("amdhsa.kernels", [])]
            mine = [s for s in syms if s in want]
            if not mine:
                continue
            obj = os.path.join(tmp, f"co{i}.o")
            with open(obj, "wb") as f:
                f.write(co)
            res = subprocess.run([tool, "-d", f"--mcpu={arch}", "--disassemble-symbols=" + ",".join(mine), obj],
                                 capture_output=True, text=True, check=True)
            current = None
            for line in res.stdout.splitlines():
                if line.endswith(">:"):
                    current = line[line.index("<") + 1:-2]
                    counts.setdefault(current, 0)
                elif current and "scratch_" in line:
                    counts[current] += 1
    return counts


def print_kernel_metadata(match: str = "", path: Optional[str] = None, file=None) -> List[Dict]:
    """Print the registers, LDS, scratch and spills of every kernel whose
    demangled name contains `match` (all kernels for ''), one line each,
    and return the rows."""
    rows = [r for r in kernel_metadata(path) if match in r["name"]]
    lds_cu = 160 * 1024
    for r in rows:
        print(f"{r['name'][:110]:110s}  VGPR {r['vgpr']:3d}  AGPR {r['agpr']:3d}  SGPR {r['sgpr']:3d}  "
              f"LDS {r['lds_bytes']:6d} B ({100.0 * r['lds_bytes'] / lds_cu:4.1f}% of a CU)  "
              f"scratch {r['scratch_bytes']:3d} B/lane  spills VGPR {r['vgpr_spills']} SGPR {r['sgpr_spills']}",
              file=file)
    return rows
