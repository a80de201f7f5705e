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
build produced) and simulates the LGKM counter along every control-flow path:
LDS requests complete in order, so `s_waitcnt lgkmcnt(N)` retires all but the
newest N; a scalar memory request (which completes out of order) makes a
partial wait retire nothing.  The queue of outstanding requests is carried
across branches to their targets (and across the loop back edges), and the
set of queues reaching each instruction is iterated to a fixed point, so a
load issued at the bottom of a loop and waited for at the top of the next
iteration is followed like any other.  Any instruction other than a later LDS
read into the same register that touches a register whose LDS load has not
been retired on some path is reported.  Only the library's own kernels (names
in the ``otx`` namespace) are checked.
"""

from __future__ import annotations

import pathlib
import re
import shutil
import struct
import subprocess
import tempfile

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


_ADDR = re.compile(r"//\s*([0-9A-Fa-f]+):")
_TARGET = re.compile(r"<([^>+]+)\+0x([0-9a-fA-F]+)>")
_MAX_STATES = 32  # queues kept per instruction before they are widened into one


def _functions(text: str, namespace: str):
    """{name: (start address, [(address, op, args, text, branch target or None)])}."""
    funcs: dict[str, tuple[int, list]] = {}
    fn = None
    for raw in text.splitlines():
        m = re.match(r"^([0-9a-f]+) <([^>]+)>:", raw)
        if m:
            fn = m.group(2)
            funcs[fn] = (int(m.group(1), 16), [])
            continue
        if fn is None or namespace not in fn:
            continue
        s = raw.split("//")[0].strip()
        if not s or s.endswith(":"):
            continue
        start, body = funcs[fn]
        am = _ADDR.search(raw)
        addr = int(am.group(1), 16) if am else (body[-1][0] + 4 if body else start)
        tm = _TARGET.search(raw)
        target = start + int(tm.group(2), 16) if (tm and tm.group(1) == fn) else None
        op, _, args = s.partition(" ")
        body.append((addr, op, args, s, target))
    return {f: v for f, v in funcs.items() if namespace in f}


def _successors(k: int, body: list) -> list[int]:
    addr, op, _, _, target = body[k]
    if op.startswith("s_endpgm") or op in ("s_setpc_b64", "s_trap"):
        return []
    index = {a: i for i, (a, *_rest) in enumerate(body)} if target is not None else {}
    succ = []
    if op.startswith(("s_branch", "s_cbranch")):
        if target is None or target not in index:
            raise ValueError(f"branch without a resolvable target: {body[k][3]}")
        succ.append(index[target])
        if op.startswith("s_branch"):
            return succ
    if k + 1 < len(body):
        succ.append(k + 1)
    return succ


def _step(state: tuple, op: str, args: str):
    """(hazard registers, next state) of one instruction on one queue state.
    A state is a tuple of (registers, is_scalar) requests in issue order."""
    if op == "s_waitcnt":
        lm = re.search(r"lgkmcnt\((\d+)\)", args)
        if lm:
            n = int(lm.group(1))
            if n == 0:
                return set(), ()
            if not any(smem for _, smem in state):
                state = state[max(0, len(state) - n):]
        return set(), state
    parts = [p.strip() for p in args.split(",")] if args else []
    touched = set().union(*map(_regs, parts)) if parts else set()
    pending = set().union(*[r for r, _ in state]) if state else set()
    is_lds_read = op.startswith("ds_read") or op.startswith("ds_load")
    dst = _regs(parts[0]) if (is_lds_read and parts) else set()
    bad = (touched - dst) & pending if is_lds_read else touched & pending
    if op.startswith("ds_"):
        writes_reg = not (op.startswith("ds_write") or op.startswith("ds_store"))
        state = state + ((frozenset(_regs(parts[0])) if (writes_reg and parts) else frozenset(), False),)
    elif op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_scratch_load")):
        state = state + ((frozenset(), True),)
    return bad, _normal(state)


def _normal(state: tuple) -> tuple:
    """Drop LDS requests without a register destination (writes) that are older
    than every other request: a wait retires the oldest first, so they never
    decide whether a later load has retired.  This keeps loops that store to
    LDS without waiting from growing the queue without bound."""
    k = 0
    while k < len(state) and not state[k][0] and not state[k][1]:
        k += 1
    return state[k:]


def _widen(states) -> tuple:
    """One queue covering every given one: all their registers pending until
    lgkmcnt(0) (a scalar entry makes partial waits retire nothing)."""
    regs = frozenset().union(*[r for st in states for r, _ in st])
    return ((regs, True),)


def scan(text: str, namespace: str = "otx") -> dict[str, list[tuple[str, list[str]]]]:
    """{function: [(instruction, registers touched while their LDS load is in flight)]}."""
    hazards: dict[str, list] = {}
    for fn, (_, body) in _functions(text, namespace).items():
        if not body:
            continue
        seen: list[set] = [set() for _ in body]
        work = [(0, ())]
        found: dict[int, set] = {}
        while work:
            k, st = work.pop()
            if st in seen[k]:
                continue
            if len(seen[k]) >= _MAX_STATES:
                st = _widen(list(seen[k]) + [st])
                if st in seen[k]:
                    continue
            seen[k].add(st)
            _, op, args, txt, _ = body[k]
            bad, nxt = _step(st, op, args)
            if bad:
                found.setdefault(k, set()).update(bad)
            for j in _successors(k, body):
                work.append((j, nxt))
        if found:
            hazards[fn] = [(body[k][3], sorted(found[k])) for k in sorted(found)]
    return hazards


def check_library(lib_path: str | pathlib.Path) -> dict[str, list]:
    return scan(disassemble(lib_path))
