"""ctypes binding of the C ABI in include/clove/gemm_c.h (libclove_gemm.so).

The library is the HIP product path; there is no fallback.  Loading fails
loudly when the shared object has not been built.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libclove_gemm.so")

CLOVE_OK = 0
CLOVE_ERR_NULL_POINTER = 1
CLOVE_ERR_INVALID_DIM = 2
CLOVE_ERR_INVALID_ARG = 3
CLOVE_ERR_ALIASING = 4
CLOVE_ERR_OUT_OF_MEMORY = 5
CLOVE_ERR_LAUNCH = 6
CLOVE_ERR_NO_DEVICE = 7
CLOVE_ERR_WORKSPACE = 8
CLOVE_ERR_SCRATCH_LIMIT = 9

CLOVE_WORKSPACE_MIN_BYTES = 65536
CLOVE_NOALLOC_SCRATCH_BYTES = 65 << 20

CLOVE_INT4_GROUPWISE = 0
CLOVE_INT4_REFERENCE_LITERAL = 1
CLOVE_INT8_EXACT = 0
CLOVE_INT8_REFERENCE_LITERAL = 1

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
I8 = ctypes.c_int8

# name -> argtypes (every entry point declared in include/clove/gemm_c.h)
SIGNATURES = {
    "clove_status_string": ([I], ctypes.c_char_p),
    "clove_abi_version": ([], I),
    "clove_gemm_fp16": ([P, P, P, I, I, I, F, F, P], I),
    "clove_gemm_fp16_batched": ([P, P, P, I, I, I, I, F, F, P], I),
    "clove_gemm_fp16_noalloc": ([P, P, P, I, I, I, F, F, P], I),
    "clove_gemm_int8": ([P, P, P, I, I, I, F, I8, F, I8, P], I),
    "clove_gemm_int8_ex": ([P, P, P, I, I, I, F, I8, F, I8, I, P], I),
    "clove_gemm_int8_rowcol": ([P, P, P, P, P, I, I, I, I8, I8, P], I),
    "clove_gemm_int8_acc32": ([P, P, P, I, I, I, I8, I8, P], I),
    "clove_gemm_int4_group_acc32": ([P, P, P, P, P, I, I, I, P], I),
    "clove_gemm_int4": ([P, P, P, P, P, P, P, I, I, I, P], I),
    "clove_gemm_int4_ex": ([P, P, P, P, P, P, P, I, I, I, I, P], I),
    "clove_gemm_w4a16": ([P, P, P, P, P, I, I, I, F, F, P], I),
    "clove_swiglu": ([P, P, P, I, P], I),
    "clove_swiglu_fused": ([P, P, P, P, I, I, I, P], I),
    "clove_w4a16_swiglu": ([P, P, P, P, P, I, I, I, P], I),
    "clove_workspace_bind": ([P, ctypes.c_size_t], I),
    "clove_workspace_query_begin": ([], I),
    "clove_workspace_query_end": ([], ctypes.c_size_t),
    "clove_release_scratch": ([], I),
}

_lib = None


class CloveError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {status_string(status)}")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().clove_status_string(int(status)).decode()


def check(status: int, where: str) -> None:
    if status != CLOVE_OK:
        raise CloveError(status, where)
