"""The built library never touches a register while an LDS load into it is in flight.

The matrix chains issue their LDS reads by hand and count them with explicit
lgkmcnt waits, which the compiler cannot see; a register copy placed between
such a read and its wait takes the register's old value whenever the load is
slow.  isa_check simulates the LGKM counter over the disassembled library.
The checker itself is pinned on hand-written listings: the same copy is a
hazard before the wait and fine after it, and a scalar load in flight makes a
partial wait retire nothing.
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
