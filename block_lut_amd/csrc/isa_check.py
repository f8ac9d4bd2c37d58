"""Hazard check over the gfx950 code of liblutmoe's own objects.

The kernels issue their LDS-DMA loads (global_load_lds_*) as inline asm, so the
compiler's hazard recognizer does not look at them.  On gfx950 (a GFX9 target) a
VMEM instruction that reads an SGPR written by a VALU instruction (v_readlane,
v_readfirstlane, a VOP3 carry-out, a compare) needs 5 wait states in between:
the compiler puts `s_nop 4` in front of its own loads in that case.  Without
them the load may use the SGPR's old value as its base address.

This module disassembles the device code object embedded in each built object
(llvm-objcopy, clang-offload-bundler, llvm-objdump from the ROCm toolchain) and
walks back from every LDS-DMA load along every path into it (fall-through and
branches), for 5 wait states, looking for a VALU write of an SGPR the load reads
(its base pair and M0).

    python -m block_lut_amd.csrc.isa_check      # checks block_lut_amd/_build/*.o
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
WAIT_STATES = 5

_INSN = re.compile(r"^\s+([a-z_0-9]+)(.*?)\s*//\s*([0-9A-Fa-f]+):")
_FUNC = re.compile(r"^([0-9a-f]+) <(.+)>:")
_TARGET = re.compile(r"<(.+)\+0x([0-9a-f]+)>\s*$")
_SPAIR = re.compile(r"^s\[(\d+):(\d+)\]$")
_SREG = re.compile(r"^s(\d+)$")


def _sregs(tok: str) -> set:
    tok = tok.strip()
    m = _SPAIR.match(tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    if _SREG.match(tok) or tok in ("m0", "vcc"):
        return {tok}
    return set()


def _operands(rest: str) -> list:
    return [o.strip() for o in rest.split(",")] if rest.strip() else []


def _valu_sgpr_defs(mnem: str, ops: list) -> set:
    """SGPRs (and M0) a VALU instruction writes: its first operand when that is
    scalar (v_readlane, v_readfirstlane, v_cmp_*_e64), and the second one of the
    VOP3 forms with a scalar carry or condition output."""
    if not mnem.startswith("v_") or not ops:
        return set()
    defs = _sregs(ops[0])
    if len(ops) > 1 and ("_co_" in mnem or mnem.startswith(("v_mad_u64_u32", "v_mad_i64_i32", "v_div_scale"))):
        defs |= _sregs(ops[1])
    if mnem.startswith("v_cmp") and not mnem.endswith("_e64"):
        defs.add("vcc")
    return defs


def disassemble(obj: str) -> str:
    """llvm-objdump text of the gfx950 code object inside a built object (or of a
    code object file)."""
    with tempfile.TemporaryDirectory() as td:
        fat = os.path.join(td, "fatbin")
        co = os.path.join(td, "co")
        r = subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(td, "x")],
                           capture_output=True, text=True)
        if r.returncode != 0 or not os.path.exists(fat):
            return ""
        r = subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--targets={TARGET}",
                            f"--input={fat}", f"--output={co}"], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"clang-offload-bundler failed on {obj}:\n{r.stderr}")
        r = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"llvm-objdump failed on {obj}:\n{r.stderr}")
        return r.stdout


def find_hazards(text: str) -> list:
    """(function, address, offending VALU, load) for every LDS-DMA load with a
    VALU write of one of its SGPRs fewer than WAIT_STATES wait states earlier on
    some path."""
    funcs = {}
    insns = []            # (func, addr, mnemonic, operands)
    cur = None
    for line in text.splitlines():
        m = _FUNC.match(line)
        if m:
            cur = m.group(2)
            funcs[cur] = int(m.group(1), 16)
            continue
        m = _INSN.match(line)
        if m and cur is not None:
            rest = m.group(2)
            tgt = _TARGET.search(line)
            insns.append((cur, int(m.group(3), 16), m.group(1), _operands(rest), tgt))
    index = {a: i for i, (_, a, _, _, _) in enumerate(insns)}
    preds_by_branch = {}
    for i, (f, a, mn, ops, tgt) in enumerate(insns):
        if mn.startswith(("s_branch", "s_cbranch")) and tgt and tgt.group(1) in funcs:
            dest = funcs[tgt.group(1)] + int(tgt.group(2), 16)
            preds_by_branch.setdefault(dest, []).append(i)

    def preds(i):
        out = list(preds_by_branch.get(insns[i][1], []))
        if i > 0 and insns[i - 1][0] == insns[i][0] and not insns[i - 1][2].startswith(
                ("s_branch", "s_endpgm", "s_setpc")):
            out.append(i - 1)
        return out

    hits = []
    for i, (f, a, mn, ops, _) in enumerate(insns):
        if not mn.startswith("global_load_lds"):
            continue
        used = {"m0"}
        for o in ops[1:]:
            used |= _sregs(o)
        stack = [(p, 0) for p in preds(i)]
        seen = set()
        while stack:
            j, ws = stack.pop()
            if ws >= WAIT_STATES or (j, ws) in seen:
                continue
            seen.add((j, ws))
            _, aj, mj, oj, _ = insns[j]
            if _valu_sgpr_defs(mj, oj) & used:
                hits.append((f, a, f"{mj} {', '.join(oj)}", f"{mn} {', '.join(ops)}"))
                break
            step = int(oj[0], 0) + 1 if mj == "s_nop" and oj else 1
            stack.extend((p, ws + step) for p in preds(j))
    return hits


def check_objects(objs) -> list:
    hits = []
    for o in objs:
        text = disassemble(o)
        hits += [(os.path.basename(o),) + h for h in find_hazards(text)]
    return hits


def check_build(build_dir: str | None = None) -> list:
    build_dir = build_dir or os.path.join(PKG, "_build")
    return check_objects(sorted(glob.glob(os.path.join(build_dir, "*.o"))))


if __name__ == "__main__":
    found = check_build()
    for h in found:
        print(*h, sep="  |  ")
    print(f"{len(found)} hazard(s)")
    sys.exit(1 if found else 0)
