"""The wait-state scan of the built kernels (clove_compute_amd/hazards.py).

The kernels issue their LDS DMAs as inline assembly, which the compiler's
hazard recognizer does not look into.  A VALU write of an SGPR (the compiler
restoring a spilled SGPR with v_readlane_b32) followed by such a DMA reading
that SGPR as its buffer resource within fewer than 5 wait states made the
INT4 partials kernel read weight rows as zeros and fault the GPU; the scan
finds exactly that pattern, and build() fails on it.
"""
import glob
import os

import pytest

from clove_compute_amd import hazards

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _listing(body: str) -> str:
    return "\n0000000000001000 <_Z6kernelv>:\n" + "\n".join("\t" + l for l in body.strip().splitlines()) + "\n"


def test_valu_sgpr_write_before_dma_is_found():
    text = _listing("""
        v_readlane_b32 s46, v174, 10
        v_readlane_b32 s47, v174, 11
        s_mov_b32 m0, s2
        s_nop 0
        buffer_load_dword v2, s[44:47], s0 offen lds
    """)
    found = hazards.scan(text)
    assert len(found) == 2 and all("v_readlane_b32" in f for f in found)
    assert "after 2 wait states" in found[0] or "after 2 wait states" in found[1]


def test_five_wait_states_clear_it():
    text = _listing("""
        v_readlane_b32 s47, v174, 11
        s_mov_b32 m0, s2
        s_nop 4
        buffer_load_dword v2, s[44:47], s0 offen lds
    """)
    assert hazards.scan(text) == []


def test_m0_write_right_before_lds_dma_is_found():
    text = _listing("""
        s_add_i32 m0, s23, s1
        buffer_load_dwordx4 v48, s[60:63], s0 offen lds
    """)
    found = hazards.scan(text)
    assert len(found) == 1 and "m0" in found[0]
    # an ordinary load does not read M0
    assert hazards.scan(_listing("""
        s_add_i32 m0, s23, s1
        buffer_load_dwordx4 v[0:3], v48, s[60:63], s0 offen
    """)) == []


def test_sgpr_not_read_by_the_load_is_not_flagged():
    text = _listing("""
        v_readfirstlane_b32 s9, v1
        s_mov_b32 m0, s2
        s_nop 0
        buffer_load_dword v2, s[44:47], s0 offen lds
    """)
    assert hazards.scan(text) == []


def test_built_library_has_no_hazards():
    objs = sorted(glob.glob(os.path.join(ROOT, "clove_compute_amd", "_build", "*.hip.o")))
    if not objs:
        pytest.skip("library not built")
    assert hazards.report(objs) == []
