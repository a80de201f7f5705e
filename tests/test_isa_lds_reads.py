"""The built library never touches a register while an LDS load into it is in flight.

The matrix chains issue their LDS reads by hand and count them with explicit
lgkmcnt waits, which the compiler cannot see; a register copy placed between
such a read and its wait takes the register's old value whenever the load is
slow.  isa_check simulates the LGKM counter over the disassembled library,
along every control-flow path.  The checker itself is pinned on hand-written
listings: the same copy is a hazard before the wait and fine after it, a
scalar load in flight makes a partial wait retire nothing, a load issued at
the bottom of a loop is still in flight at the top of the next iteration, and
a load retired on one arm of a branch but not on the other is in flight where
the arms join.
"""

from __future__ import annotations

import pathlib

import pytest

from open_transformers_amd import isa_check

LIB = pathlib.Path(isa_check.__file__).resolve().parent / "libotx_attn.so"


def _listing(body: str, name: str = "_ZN3otx4testEv") -> str:
    return f"0000000000001000 <{name}>:\n" + "\n".join("\t" + line for line in body.strip().splitlines()) + "\n"


def test_checker_flags_copy_before_wait():
    text = _listing("""
ds_read_u16_d16_hi v10, v1 offset:0
ds_read_u16_d16_hi v11, v2 offset:0
v_mov_b32_e32 v20, v10
s_waitcnt lgkmcnt(1)
v_mfma_f32_32x32x1_2b_f32 a[0:31], v20, v11, a[0:31]
""")
    hz = isa_check.scan(text)
    assert list(hz) == ["_ZN3otx4testEv"]
    assert hz["_ZN3otx4testEv"][0][1] == ["v10"]
    # the MFMA reads v11, whose load lgkmcnt(1) has not retired either
    assert hz["_ZN3otx4testEv"][1][1] == ["v11"]


def test_checker_accepts_copy_after_its_wait():
    text = _listing("""
ds_read_u16_d16_hi v10, v1 offset:0
ds_read_u16_d16_hi v11, v2 offset:0
s_waitcnt lgkmcnt(1)
v_mov_b32_e32 v20, v10
s_waitcnt lgkmcnt(0)
v_mfma_f32_32x32x1_2b_f32 a[0:31], v20, v11, a[0:31]
ds_read_u16_d16_hi v10, v1 offset:2
""")
    assert isa_check.scan(text) == {}


def test_checker_partial_wait_with_scalar_load_in_flight_retires_nothing():
    text = _listing("""
ds_read_b32 v10, v1
s_memtime s[4:5]
ds_read_b32 v11, v2
s_waitcnt lgkmcnt(1)
v_add_f32_e32 v12, v10, v10
""")
    assert isa_check.scan(text)["_ZN3otx4testEv"][0][1] == ["v10"]


def _addressed(name: str, start: int, lines: list[str]) -> str:
    """A listing in llvm-objdump's layout: each instruction with its address
    comment, branch targets as <name+0xOFF>."""
    out = [f"{start:016x} <{name}>:"]
    for i, ins in enumerate(lines):
        out.append(f"\t{ins:<50} // {start + 4 * i:012X}: 00000000")
    return "\n".join(out) + "\n"


def _loop(wait_at_top: bool) -> str:
    name = "_ZN3otx4loopEv"
    top = 3  # index of the loop's first instruction
    body = ["s_mov_b32 s0, 4", "ds_read_b32 v10, v1", "s_waitcnt lgkmcnt(0)"]
    body += ["s_waitcnt lgkmcnt(0)"] if wait_at_top else ["s_nop 0"]
    body += ["v_add_f32_e32 v12, v10, v10", "ds_read_b32 v10, v1", "s_sub_u32 s0, s0, 1",
             f"s_cbranch_scc1 -5 <{name}+0x{4 * top:x}>", "s_endpgm"]
    return _addressed(name, 0x1000, body)


def test_checker_follows_the_loop_back_edge():
    """In program order the load at the loop's bottom is never used before
    s_endpgm; along the back edge it is in flight when the next iteration's
    v_add reads v10."""
    hz = isa_check.scan(_loop(wait_at_top=False))
    assert hz == {"_ZN3otx4loopEv": [("v_add_f32_e32 v12, v10, v10", ["v10"])]}
    assert isa_check.scan(_loop(wait_at_top=True)) == {}


def test_checker_joins_branch_arms():
    name = "_ZN3otx4diamondEv"
    body = ["ds_read_b32 v10, v1", "s_cbranch_scc1 3 <%s+0x14>" % name, "s_waitcnt lgkmcnt(0)",
            "v_mov_b32_e32 v11, 0", "s_branch 0 <%s+0x14>" % name, "v_mov_b32_e32 v12, v10", "s_endpgm"]
    hz = isa_check.scan(_addressed(name, 0x2000, body))
    assert hz == {name: [("v_mov_b32_e32 v12, v10", ["v10"])]}
    body[1] = "s_nop 0"  # no branch: the wait always runs first
    assert isa_check.scan(_addressed(name, 0x2000, body)) == {}


def test_checker_ignores_other_namespaces():
    text = _listing("""
ds_read_b32 v10, v1
v_mov_b32_e32 v20, v10
""", name="_ZN7rocprim6kernelEv")
    assert isa_check.scan(text) == {}


@pytest.mark.skipif(not LIB.exists(), reason="libotx_attn.so is not built")
def test_built_library_has_no_register_touched_in_flight():
    text = isa_check.disassemble(LIB)
    assert "attn_dkdv_bf16_kb2_kernel" in text and "attn_fwd_bf16_kernel" in text
    hazards = isa_check.scan(text)
    assert hazards == {}, {fn: v[:3] for fn, v in hazards.items()}
