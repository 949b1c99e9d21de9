"""Builds the gfx950 GEMM library libclove_gemm.so in-tree with hipcc.

Each .hip source under csrc/ is compiled to an object for gfx950 only, then
linked into clove_compute_amd/lib/libclove_gemm.so.  Objects are rebuilt when
their source or any header is newer (force=True rebuilds everything).  The
build then reads every kernel's register and scratch use from the code objects
(resources.py) and fails if a kernel outside the unaligned fallbacks spills,
and scans their disassembly for memory instructions issued without the wait
states a gfx9 hazard requires (hazards.py).
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libclove_gemm.so")
# diagnostics for bench.py --floor (not part of the GEMM C-ABI)
DIAG_SRC = os.path.join(CSRC, "diag")
DIAG_LIB = os.path.join(LIBDIR, "libclove_diag.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-munsafe-fp-atomics",
    # every fused multiply-add is written as fmaf(); no implicit contraction
    # (which would also fuse fp32 multiplies with the fp16 narrowing)
    "-ffp-contract=off",
    # keep hipcc from emitting packed fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


# per-source additions: the INT4-weight GEMMs keep their per-group MFMA sums in
# VGPRs (the group fold reads every one of them; in AGPRs each read would be a
# separate v_accvgpr_read)
EXTRA = {"i4w_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "i4i4_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _headers_mtime():
    hs = glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(ROOT, "include", "clove", "*.h"))
    return max((os.path.getmtime(h) for h in hs), default=0.0)


def _compile(src: str, force: bool) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if (not force and os.path.exists(obj)
            and os.path.getmtime(obj) >= max(os.path.getmtime(src), _headers_mtime())):
        return obj
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}")
    os.replace(obj + ".tmp", obj)
    return obj


def build(force: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB + ".tmp", *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libclove_gemm.so failed")
    os.replace(LIB + ".tmp", LIB)
    dsrcs = sorted(glob.glob(os.path.join(DIAG_SRC, "*.hip")))
    dobjs = [_compile(s, force) for s in dsrcs]
    if dobjs:
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", DIAG_LIB + ".tmp", *dobjs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("link of libclove_diag.so failed")
        os.replace(DIAG_LIB + ".tmp", DIAG_LIB)
    # no kernel that an aligned call can reach may spill registers to scratch
    from clove_compute_amd import hazards, resources
    resources.check(objs + dobjs)
    # every inline-asm memory instruction has its wait states
    hazards.check(objs + dobjs)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
