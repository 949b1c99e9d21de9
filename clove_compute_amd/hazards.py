"""Wait-state check of the hand-placed memory instructions in the built gfx950 objects.

The kernels issue their LDS DMAs (`buffer_load_dword[x4] ... lds`) as inline
assembly, so the compiler's hazard recognizer does not know what they are and
inserts no wait states before them.  Two gfx9 hazards apply to them (the
compiler inserts exactly these wait states before its own LDS DMAs and VMEM
instructions):

  * a VALU instruction that writes an SGPR (v_readlane_b32,
    v_readfirstlane_b32, a v_cmp with an SGPR destination, ...) followed by a
    VMEM instruction that reads that SGPR as its buffer resource or soffset:
    5 wait states.  With fewer, the VMEM instruction may read the SGPR's old
    value: a stale resource word sends the load to the wrong address or
    range (wrong data, or a memory fault).
  * an SALU write of M0 followed by an LDS DMA, which takes its LDS address
    from M0: 1 wait state.

`scan(text)` walks each kernel's disassembly in program order and reports
every VMEM / LDS-DMA instruction with fewer wait states than that behind the
writer (an instruction counts one wait state, `s_nop n` counts n + 1).  A
branch target is not followed back to its other predecessors: the scan covers
the straight-line code in front of each instruction, which is where the
inline assembly's operands are set up.

build() calls check(): it fails when any kernel has such an instruction.
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
OBJ = os.path.join(HERE, "_build")
LLVM = "/opt/rocm/llvm/bin"

VALU_SGPR_VMEM = 5
SALU_M0_LDSDMA = 1

_VMEM = re.compile(r"^(buffer|global|flat|scratch)_")
_INSN = re.compile(r"^\s+([a-z_][a-z0-9_]*)(\s+[^/]*?)?\s*(//.*)?$")
_LABEL = re.compile(r"^([0-9a-f]+ )?<?([A-Za-z_.$][\w.$]*)>?:\s*$")


def _sgprs(tok: str) -> set[int]:
    tok = tok.strip()
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return {int(m.group(1))}
    return set()


def _operands(rest: str) -> list[str]:
    rest = (rest or "").strip()
    return [o.strip() for o in rest.split(",")] if rest else []


def scan(text: str) -> list[str]:
    """Hazards in one disassembly listing (llvm-objdump -d); one line each."""
    found = []
    kernel = "?"
    window: list[tuple[str, list[str]]] = []  # preceding instructions, newest last
    for line in text.splitlines():
        lm = _LABEL.match(line)
        if lm:
            if lm.group(1):  # a symbol: a new function
                kernel = lm.group(2)
                window = []
            continue
        m = _INSN.match(line)
        if not m:
            continue
        op, ops = m.group(1), _operands(m.group(2))
        if _VMEM.match(op):
            # the SGPR operands: the resource and soffset of a buffer access,
            # the saddr of a global one (every s operand after the VGPR ones)
            reads = set()
            for o in ops:
                for t in o.split():
                    reads |= _sgprs(t)
            lds_dma = op.startswith(("buffer_load", "global_load_lds")) and any(
                t == "lds" for o in ops for t in o.split())
            ws = 0
            for pop, pops in reversed(window):
                if ws >= VALU_SGPR_VMEM:
                    break
                if pop == "s_nop":
                    ws += int(pops[0], 0) + 1 if pops else 1
                    continue
                dst = pops[0] if pops else ""
                if pop.startswith("v_") and _sgprs(dst) & reads:
                    found.append(f"{kernel}: {pop} {dst} then {op} {', '.join(ops)} "
                                 f"after {ws} wait states (needs {VALU_SGPR_VMEM})")
                if lds_dma and ws < SALU_M0_LDSDMA and pop.startswith("s_") and dst == "m0":
                    found.append(f"{kernel}: {pop} m0 then {op} {', '.join(ops)} "
                                 f"after {ws} wait states (needs {SALU_M0_LDSDMA})")
                ws += 1
        window.append((op, ops))
        if len(window) > 16:
            del window[0]
    return found


def _disassemble(obj: str) -> list[str]:
    with tempfile.TemporaryDirectory() as td:
        # llvm-objdump writes the bundles next to its input: work on a copy
        src = os.path.join(td, os.path.basename(obj))
        with open(obj, "rb") as f, open(src, "wb") as g:
            g.write(f.read())
        subprocess.run([os.path.join(LLVM, "llvm-objdump"), "--offloading", src], check=True,
                       capture_output=True, text=True)
        return [subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", co],
                               check=True, capture_output=True, text=True).stdout
                for co in glob.glob(src + ".*") if "amdgcn" in co]


def report(objs: list[str] | None = None) -> list[str]:
    objs = objs if objs is not None else sorted(glob.glob(os.path.join(OBJ, "*.hip.o")))
    out = []
    for o in objs:
        for text in _disassemble(o):
            out += [f"{os.path.basename(o)}: {h}" for h in scan(text)]
    return out


def check(objs: list[str] | None = None) -> None:
    bad = report(objs)
    if bad:
        raise RuntimeError(f"{len(bad)} memory instructions without their wait states:\n  " +
                           "\n  ".join(bad[:40]))


if __name__ == "__main__":
    import sys
    bad = report()
    print("\n".join(bad))
    print(f"{len(bad)} hazards")
    sys.exit(1 if bad else 0)
