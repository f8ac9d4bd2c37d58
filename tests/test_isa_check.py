"""The build's ISA check for the inline-asm LDS-DMA loads (block_lut_amd/csrc/isa_check.py):
on gfx950 a VMEM instruction that reads an SGPR written by a VALU instruction needs 5
wait states in between, which the compiler does not insert in front of inline asm.

The checker is run on hand-written disassembly (each case built so that a plausible
mistake -- counting s_nop N as N wait states, ignoring a branch into the load, taking a
VALU read of an SGPR for a write -- fails one of them) and on the built library's own
objects when they are there."""
import glob
import os

import pytest

from block_lut_amd.csrc import isa_check as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _text(lines, base=0x1000):
    out = [f"{base:016x} <kern>:"]
    a = base
    for ln in lines:
        if isinstance(ln, tuple):          # (instruction, branch target offset)
            ln, tgt = ln
            out.append(f"\t{ln:<58}// {a:012X}: BF850000 <kern+0x{tgt:x}>")
        else:
            out.append(f"\t{ln:<58}// {a:012X}: 00000000")
        a += 4
    return "\n".join(out)


DMA = "global_load_lds_dword v2, s[6:7]"


@pytest.mark.parametrize("lines, n", [
    (["v_readlane_b32 s7, v255, 3", DMA], 1),
    (["v_readlane_b32 s7, v255, 3", "s_nop 4", DMA], 0),
    (["v_readlane_b32 s7, v255, 3", "s_nop 3", DMA], 1),                 # 4 wait states
    (["v_readfirstlane_b32 s6, v1", "s_add_i32 s8, s8, 1", "s_mov_b32 s9, 0", "s_nop 1", DMA], 1),
    (["v_readfirstlane_b32 s6, v1", "s_add_i32 s8, s8, 1", "s_mov_b32 s9, 0", "s_nop 2", DMA], 0),
    (["v_add_u32_e32 v1, s6, v2", DMA], 0),                               # a VALU read of s6
    (["v_cmp_eq_u32_e64 s[6:7], v1, v2", DMA], 1),                       # compare into s[6:7]
    (["v_add_co_u32_e64 v1, s[6:7], v2, v3", DMA], 1),                   # carry out into s[6:7]
    (["v_readfirstlane_b32 m0, v4", DMA], 1),                            # M0 from a VALU
    (["s_mov_b32 m0, s10", DMA], 0),                                     # M0 from SALU
    (["v_readlane_b32 s6, v255, 2", "s_branch 5", DMA], 0),             # not a predecessor
])
def test_straight_line(lines, n):
    assert len(C.find_hazards(_text(lines))) == n


def test_branch_into_load():
    # the fall-through path has its 5 wait states, the branch from the top of the
    # function reaches the load one wait state after the VALU write
    lines = ["v_readlane_b32 s7, v255, 3", ("s_cbranch_scc1 4", 0x18), "s_nop 4", "s_nop 4", "s_nop 4",
             "s_mov_b32 s0, 0", DMA]
    # (the branch targets offset 0x18: the load)
    assert len(C.find_hazards(_text(lines))) == 1
    lines[1] = ("s_cbranch_scc1 4", 0x10)       # now into the s_nop run instead
    assert len(C.find_hazards(_text(lines))) == 0


def test_built_objects_clean():
    objs = sorted(glob.glob(os.path.join(ROOT, "block_lut_amd", "_build", "*.o")))
    if not objs or not os.path.exists(C.LLVM):
        pytest.skip("library objects not built here")
    assert C.check_objects(objs) == []
