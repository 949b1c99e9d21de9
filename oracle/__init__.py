"""CPU oracle for the Clove Compute GEMM hot path -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``liboracle.so`` (built from ``clove_oracle.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or as the timed CPU baseline; the product library never calls it.

Half-precision arrays cross the boundary as ``numpy.float16`` (bit-identical
to the uint16 patterns the C code takes).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

GROUP = 128


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        F = ctypes.c_float
        D = ctypes.c_double
        I64 = ctypes.c_int64
        sig = {
            "oracle_f32_to_f16_array": ([P, P, I64], None),
            "oracle_f16_to_f32_array": ([P, P, I64], None),
            "oracle_gemm_fp16_rows": ([P, P, P, I, I, I, F, F, I, I], None),
            "oracle_gemm_fp16": ([P, P, P, I, I, I, F, F], None),
            "oracle_gemm_fp16_rows_mt": ([P, P, P, I, I, I, F, F, I, I, I], I),
            "oracle_gemm_fp16_f64": ([P, P, P, P, I, I, I, D, D], None),
            "oracle_gemm_fp16_batched": ([P, P, P, I, I, I, I, F, F], None),
            "oracle_gemm_int8": ([P, P, P, P, I, I, I, F, ctypes.c_int8, F, ctypes.c_int8], None),
            "oracle_gemm_int8_literal": ([P, P, P, P, I, I, I, F, ctypes.c_int8, F, ctypes.c_int8], None),
            "oracle_gemm_int8_rowcol": ([P, P, P, P, P, P, I, I, I, ctypes.c_int8, ctypes.c_int8], None),
            "oracle_gemm_int4_literal": ([P, P, P, P, P, I, I, I], None),
            "oracle_gemm_int4_groupwise": ([P, P, P, P, P, P, P, P, P, I, I, I], None),
            "oracle_w4a16": ([P, P, P, P, P, P, P, I, I, I, D, D], None),
            "oracle_swiglu": ([P, P, P, I64], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# conversions
# --------------------------------------------------------------------------
def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


# --------------------------------------------------------------------------
# GEMMs
# --------------------------------------------------------------------------
def gemm_fp16(A, B, C=None, alpha=1.0, beta=0.0, rows=None) -> np.ndarray:
    """fp16 C = alpha*A@B + beta*C with the reference's naive-kernel arithmetic.

    ``rows=(m0, m1)`` computes only that row range (others are left as in C)."""
    A = _c(A, np.float16)
    B = _c(B, np.float16)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    out = np.zeros((M, N), np.float16) if C is None else _c(C, np.float16).copy()
    m0, m1 = (0, M) if rows is None else rows
    lib().oracle_gemm_fp16_rows(_p(A), _p(B), _p(out), M, N, K, alpha, beta, m0, m1)
    return out


def gemm_fp16_mt(A, B, rows, nthreads, C=None, alpha=1.0, beta=0.0) -> np.ndarray:
    """gemm_fp16 on rows ``(m0, m1)`` with the rows spread over ``nthreads``
    POSIX threads (bit-identical to ``gemm_fp16``); other rows stay as in C."""
    A = _c(A, np.float16)
    B = _c(B, np.float16)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    out = np.zeros((M, N), np.float16) if C is None else _c(C, np.float16).copy()
    m0, m1 = rows
    r = lib().oracle_gemm_fp16_rows_mt(_p(A), _p(B), _p(out), M, N, K, alpha, beta, m0, m1, nthreads)
    if r < 0:
        raise MemoryError("oracle_gemm_fp16_rows_mt")
    return out


def gemm_fp16_f64(A, B, C=None, alpha=1.0, beta=0.0) -> np.ndarray:
    A = _c(A, np.float16)
    B = _c(B, np.float16)
    M, K = A.shape
    N = B.shape[1]
    Cin = None if C is None else _c(C, np.float16)
    out = np.empty((M, N), np.float64)
    lib().oracle_gemm_fp16_f64(_p(A), _p(B), _p(Cin), _p(out), M, N, K, alpha, beta)
    return out


def gemm_fp16_batched(A, B, C=None, alpha=1.0, beta=0.0) -> np.ndarray:
    A = _c(A, np.float16)
    B = _c(B, np.float16)
    batch, M, K = A.shape
    N = B.shape[2]
    out = np.zeros((batch, M, N), np.float16) if C is None else _c(C, np.float16).copy()
    lib().oracle_gemm_fp16_batched(_p(A), _p(B), _p(out), batch, M, N, K, alpha, beta)
    return out


def gemm_int8(A_q, B_q, A_scale, A_zero, B_scale, B_zero):
    """Returns (C fp16 [M,N], acc int32 [M,N])."""
    A_q = _c(A_q, np.int8)
    B_q = _c(B_q, np.int8)
    M, K = A_q.shape
    N = B_q.shape[1]
    C = np.empty((M, N), np.float16)
    acc = np.empty((M, N), np.int32)
    lib().oracle_gemm_int8(_p(A_q), _p(B_q), _p(C), _p(acc), M, N, K,
                           float(A_scale), int(A_zero), float(B_scale), int(B_zero))
    return C, acc


def gemm_int8_literal(A_q, B_q, A_scale, A_zero, B_scale, B_zero):
    """The reference kernel's arithmetic at any K (padded k of the last 32-wide
    tile contribute A_zero * B_zero).  Returns (C fp16 [M,N], acc int32 [M,N])."""
    A_q = _c(A_q, np.int8)
    B_q = _c(B_q, np.int8)
    M, K = A_q.shape
    N = B_q.shape[1]
    C = np.empty((M, N), np.float16)
    acc = np.empty((M, N), np.int32)
    lib().oracle_gemm_int8_literal(_p(A_q), _p(B_q), _p(C), _p(acc), M, N, K,
                                   float(A_scale), int(A_zero), float(B_scale), int(B_zero))
    return C, acc


def gemm_int8_rowcol(A_q, B_q, sa, sb, A_zero=0, B_zero=0):
    A_q = _c(A_q, np.int8)
    B_q = _c(B_q, np.int8)
    sa = _c(sa, np.float16)
    sb = _c(sb, np.float16)
    M, K = A_q.shape
    N = B_q.shape[1]
    C = np.empty((M, N), np.float16)
    acc = np.empty((M, N), np.int32)
    lib().oracle_gemm_int8_rowcol(_p(A_q), _p(B_q), _p(sa), _p(sb), _p(C), _p(acc),
                                  M, N, K, int(A_zero), int(B_zero))
    return C, acc


def gemm_int4_literal(A_q, A_scale, B_q, B_scale, M, N, K):
    A_q = _c(A_q, np.uint8)
    B_q = _c(B_q, np.uint8)
    A_scale = _c(A_scale, np.float16)
    B_scale = _c(B_scale, np.float16)
    C = np.empty((M, N), np.float16)
    lib().oracle_gemm_int4_literal(_p(A_q), _p(A_scale), _p(B_q), _p(B_scale), _p(C), M, N, K)
    return C


def gemm_int4_groupwise(A_q, A_scale, A_zero, B_q, B_scale, B_zero, M, N, K,
                        want_partials=False):
    """Returns (C fp16, out64 float64, partials int32 [M,N,G] or None)."""
    A_q = _c(A_q, np.uint8)
    B_q = _c(B_q, np.uint8)
    arrs = [_c(x, np.float16) for x in (A_scale, A_zero, B_scale, B_zero)]
    G = (K + GROUP - 1) // GROUP
    C = np.empty((M, N), np.float16)
    out64 = np.empty((M, N), np.float64)
    part = np.empty((M, N, G), np.int32) if want_partials else None
    lib().oracle_gemm_int4_groupwise(_p(A_q), _p(arrs[0]), _p(arrs[1]), _p(B_q),
                                     _p(arrs[2]), _p(arrs[3]), _p(C), _p(part),
                                     _p(out64), M, N, K)
    return C, out64, part


def w4a16(X, W_q, W_scale, W_zero, Y_in=None, alpha=1.0, beta=0.0):
    """Returns (Y fp16 [T,O], out64 float64 [T,O])."""
    X = _c(X, np.float16)
    W_q = _c(W_q, np.uint8)
    W_scale = _c(W_scale, np.float16)
    W_zero = _c(W_zero, np.float16)
    T, K = X.shape
    O = W_q.shape[0]
    Yin = None if Y_in is None else _c(Y_in, np.float16)
    Y = np.empty((T, O), np.float16)
    out64 = np.empty((T, O), np.float64)
    lib().oracle_w4a16(_p(X), _p(W_q), _p(W_scale), _p(W_zero), _p(Yin), _p(Y),
                       _p(out64), T, O, K, alpha, beta)
    return Y, out64


def swiglu(gate, up) -> np.ndarray:
    """The reference's SwiGLU (src/kernels/activations.cu:9-11, :76-134) on fp16
    gate / up of equal shape: fp16(silu(g) * u), silu in fp32."""
    g = _c(gate, np.float16)
    u = _c(up, np.float16)
    if g.shape != u.shape:
        raise ValueError("gate and up must have the same shape")
    out = np.empty(g.shape, np.float16)
    lib().oracle_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def w4a16_swiglu(X, W_q, W_scale, W_zero) -> np.ndarray:
    """H [T, I] = swiglu(gate, up), gate = fp16(X @ dequant(W[:I])^T), up likewise on
    W[I:2I]: the reference MLP's gate / up linear layers and SwiGLU
    (src/runtime/inference.cu:172-186) on one fused INT4 weight [2I, K/2] whose
    first I rows are the gate projection and the next I rows the up projection."""
    W_q = _c(W_q, np.uint8)
    I = W_q.shape[0] // 2
    if W_q.shape[0] != 2 * I:
        raise ValueError("the fused gate/up weight needs an even number of rows")
    gate, _ = w4a16(X, W_q[:I], W_scale[:I], W_zero[:I])
    up, _ = w4a16(X, W_q[I:], W_scale[I:], W_zero[I:])
    return swiglu(gate, up)
