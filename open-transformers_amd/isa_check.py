"""Static check of the built library's gfx950 code for registers read or
written while an LDS load into them is still in flight.

The matrix chains read their operands from LDS with hand-issued `ds_read_*`
instructions and wait for them with hand-counted `s_waitcnt lgkmcnt(N)`; the
compiler does not know these reads are asynchronous.  If it ever copies,
spills or reuses a destination register between the read and its wait (to
relieve register pressure, or because it moved a consumer past the next read
of the same register), the copy takes whatever the register held before the
load landed: a wrong value that appears only when the load is slow.  This
module disassembles the library (llvm-objdump, on the code object that the
build produced) and simulates the LGKM counter in program order: LDS requests
complete in order, so `s_waitcnt lgkmcnt(N)` retires all but the newest N; a
scalar memory request (which completes out of order) makes a partial wait
retire nothing.  Any instruction other than a later LDS read into the same
register that touches a register whose LDS load has not been retired is
reported.  Only the library's own kernels (names in the ``otx`` namespace) are
checked.
"""

from __future__ import annotations

import pathlib
import re
import shutil
import struct
import subprocess
import tempfile
from collections import deque

BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = b"hipv4-amdgcn-amd-amdhsa--gfx950"


def _tool(name: str) -> str:
    for cand in (f"/opt/rocm/llvm/bin/{name}", shutil.which(name)):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError(f"{name} not found (ROCm's LLVM tools are needed for the ISA check)")


def _elf_section(data: bytes, name: str) -> bytes:
    """Contents of section ``name`` of an ELF64 little-endian file."""
    if data[:4] != b"\x7fELF" or data[4] != 2 or data[5] != 1:
        raise ValueError("not an ELF64 little-endian file")
    shoff = struct.unpack_from("<Q", data, 0x28)[0]
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    def sh(i):
        return struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize)
    strtab = sh(shstrndx)
    for i in range(shnum):
        s = sh(i)
        nm_off = strtab[4] + s[0]
        nm = data[nm_off:data.index(b"\0", nm_off)].decode()
        if nm == name:
            return data[s[4]:s[4] + s[5]]
    raise ValueError(f"section {name} not found")


def code_objects(lib_path: str | pathlib.Path) -> list[bytes]:
    """The gfx950 code objects of every offload bundle in the library's .hip_fatbin."""
    fat = _elf_section(pathlib.Path(lib_path).read_bytes(), ".hip_fatbin")
    out = []
    pos = fat.find(BUNDLE_MAGIC)
    while pos >= 0:
        n = struct.unpack_from("<Q", fat, pos + 24)[0]
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fat, p)
            triple = fat[p + 24:p + 24 + tlen]
            p += 24 + tlen
            if triple == TARGET and size:
                out.append(fat[pos + off:pos + off + size])
        pos = fat.find(BUNDLE_MAGIC, pos + 24)
    if not out:
        raise ValueError("no gfx950 code object in the library")
    return out


def disassemble(lib_path: str | pathlib.Path) -> str:
    objdump = _tool("llvm-objdump")
    texts = []
    with tempfile.TemporaryDirectory() as d:
        for i, co in enumerate(code_objects(lib_path)):
            f = pathlib.Path(d) / f"co{i}.o"
            f.write_bytes(co)
            res = subprocess.run([objdump, "-d", "--mcpu=gfx950", "--no-show-raw-insn", str(f)],
                                 capture_output=True, text=True, check=True)
            texts.append(res.stdout)
    return "\n".join(texts)


_REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")


def _regs(tok: str) -> set[str]:
    out = set()
    for m in _REG.finditer(tok):
        if m.group(1):
            out.add(m.group(1) + m.group(2))
        else:
            out.update(f"{m.group(3)}{i}" for i in range(int(m.group(4)), int(m.group(5)) + 1))
    return out


def scan(text: str, namespace: str = "otx") -> dict[str, list[tuple[str, list[str]]]]:
    """{function: [(instruction, registers touched while their LDS load is in flight)]}."""
    hazards: dict[str, list] = {}
    fn = None
    q: deque = deque()  # outstanding LGKM requests in issue order: (registers, is_smem)
    for raw in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:", raw)
        if m:
            fn, q = m.group(1), deque()
            continue
        if fn is None or namespace not in fn:
            continue
        s = raw.split("//")[0].strip()
        if not s or s.endswith(":"):
            continue
        op, _, args = s.partition(" ")
        if op == "s_waitcnt":
            lm = re.search(r"lgkmcnt\((\d+)\)", args)
            if lm:
                n = int(lm.group(1))
                if n == 0:
                    q.clear()
                elif not any(smem for _, smem in q):
                    while len(q) > n:
                        q.popleft()
            continue
        if op.startswith("s_endpgm"):
            q.clear()
            continue
        parts = [p.strip() for p in args.split(",")] if args else []
        touched = set().union(*map(_regs, parts)) if parts else set()
        pending = set().union(*[r for r, _ in q]) if q else set()
        is_lds_read = op.startswith("ds_read") or op.startswith("ds_load")
        dst = _regs(parts[0]) if (is_lds_read and parts) else set()
        bad = (touched - dst) & pending if is_lds_read else touched & pending
        if bad:
            hazards.setdefault(fn, []).append((s, sorted(bad)))
        if op.startswith("ds_"):
            writes_reg = not (op.startswith("ds_write") or op.startswith("ds_store"))
            q.append((_regs(parts[0]) if (writes_reg and parts) else set(), False))
        elif op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_scratch_load")):
            q.append((set(), True))
    return hazards


def check_library(lib_path: str | pathlib.Path) -> dict[str, list]:
    return scan(disassemble(lib_path))
