"""Per-kernel register and scratch report of the built gfx950 objects.

Reads the AMDGPU code-object metadata (the `.amdhsa.kernels` note) of every
object under clove_compute_amd/_build: the device code object is extracted
from each host object's offload bundle with llvm-objdump --offloading and its
notes are read with llvm-readelf.  A kernel whose private segment is not empty
spills registers to scratch memory; the HIP runtime then sizes and allocates
that scratch on the kernel's first dispatch, outside any workspace a caller
has bound.

build() calls check(): it fails when any kernel has a private segment.
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

_FIELDS = ("name", "private_segment_fixed_size", "vgpr_count", "agpr_count", "sgpr_count",
           "vgpr_spill_count", "sgpr_spill_count", "group_segment_fixed_size")


def _kernels_of(obj: str) -> list[dict]:
    with tempfile.TemporaryDirectory() as td:
        # llvm-objdump writes the bundles next to its input: work on a copy
        src = os.path.join(td, os.path.basename(obj))
        with open(obj, "rb") as f, open(src, "wb") as g:
            g.write(f.read())
        subprocess.run([os.path.join(LLVM, "llvm-objdump"), "--offloading", src], check=True,
                       capture_output=True, text=True)
        cos = [p for p in glob.glob(src + ".*") if "amdgcn" in p]
        out = []
        for co in cos:
            notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], check=True,
                                   capture_output=True, text=True).stdout
            # kernel records are the outermost "- ." list entries (argument
            # records are nested deeper)
            lines = notes.splitlines()
            items = [len(l) - len(l.lstrip()) for l in lines if re.match(r"^\s*-\s+\.", l)]
            if not items:
                continue
            top = min(items)
            cur = None
            for line in lines:
                m = re.match(r"^(\s*)(-\s+)?\.([a-z_]+):\s*(\S+)\s*$", line)
                if not m:
                    continue
                key, val = m.group(3), m.group(4)
                if m.group(2) and len(m.group(1)) == top:  # a new kernel record
                    cur = {}
                    out.append(cur)
                if cur is not None and key in _FIELDS and key not in cur:
                    cur[key] = val
        return [k for k in out if "name" in k and "private_segment_fixed_size" in k]


def report(objs: list[str] | None = None) -> list[dict]:
    objs = objs if objs is not None else sorted(glob.glob(os.path.join(OBJ, "*.hip.o")))
    rows = []
    for o in objs:
        for k in _kernels_of(o):
            k["object"] = os.path.basename(o)
            k["scratch"] = int(k["private_segment_fixed_size"])
            rows.append(k)
    return rows


def disallowed(rows: list[dict]) -> list[dict]:
    return [r for r in rows if r["scratch"] > 0]


def check(objs: list[str] | None = None) -> list[dict]:
    rows = report(objs)
    bad = disallowed(rows)
    if bad:
        lines = "\n".join(f"  {r['object']}: {r['name']} scratch {r['scratch']} B/lane, "
                          f"vgpr {r.get('vgpr_count')} agpr {r.get('agpr_count')}" for r in bad)
        raise RuntimeError("kernels spill to scratch:\n" + lines)
    return rows


if __name__ == "__main__":
    import sys
    rows = report()
    for r in rows:
        if r["scratch"] or "-v" in sys.argv:
            print(f"{r['scratch']:5d} B/lane  v{r.get('vgpr_count', '?'):>4} a{r.get('agpr_count', '?'):>4}  "
                  f"{r['object']:20s} {r['name']}")
    bad = disallowed(rows)
    print(f"{len(rows)} kernels, {sum(1 for r in rows if r['scratch'])} with scratch, "
          f"{len(bad)} not allowed")
    sys.exit(1 if bad else 0)
