"""Write the golden fixtures of the GEMM hot path: seeded small inputs and the CPU
oracle's outputs, one ``.npz`` per case (plain arrays, no pickles).

The reference ships no vectors for this path (its tests compare against live
cuBLAS on unseeded random inputs, tests/test_gemm.cu:62-112), so the fixtures are
made here from the oracle and frozen: ``tests/test_golden.py`` checks that the
oracle still reproduces them bit for bit, checks them against numpy where the
arithmetic is exact, and checks the HIP library against them on the GPU.

    python tests/golden/make_golden.py      # from the repository root
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from clove_compute_amd import quant  # noqa: E402


def _f16(a):
    return np.asarray(a).astype(np.float16)


def fp16_cases(g):
    out = {}
    # the reference test's square case at a fixture size, a ragged case with the
    # alpha / beta of its test_gemm_alpha_beta (tests/test_gemm.cu:221-243) and a
    # decode row
    for name, (M, N, K, alpha, beta) in {
        "fp16_64x64x64": (64, 64, 64, 1.0, 0.0),
        "fp16_33x17x40_alpha_beta": (33, 17, 40, 0.5, 0.25),
        "fp16_1x96x128_decode": (1, 96, 128, 1.0, 0.0),
    }.items():
        A = _f16(g.uniform(-1, 1, (M, K)))
        B = _f16(g.uniform(-1, 1, (K, N)))
        C = _f16(g.uniform(-1, 1, (M, N)))
        out[name] = dict(A=A, B=B, C_in=C, alpha=np.float32(alpha), beta=np.float32(beta),
                         C=oracle.gemm_fp16(A, B, C, alpha, beta),
                         C64=oracle.gemm_fp16_f64(A, B, C, alpha, beta))
    A = _f16(g.uniform(-1, 1, (3, 5, 40)))
    B = _f16(g.uniform(-1, 1, (3, 40, 24)))
    out["fp16_batched_3x5x24x40"] = dict(A=A, B=B, alpha=np.float32(1.0), beta=np.float32(0.0),
                                         C=oracle.gemm_fp16_batched(A, B),
                                         C64=np.stack([oracle.gemm_fp16_f64(a, b) for a, b in zip(A, B)]))
    return out


def int8_cases(g):
    M, N, K = 17, 40, 64
    A = g.integers(-127, 128, (M, K)).astype(np.int8)
    B = g.integers(-127, 128, (K, N)).astype(np.int8)
    sa, za, sb, zb = 0.0125, 3, 0.02, -2
    C, acc = oracle.gemm_int8(A, B, sa, za, sb, zb)
    out = {"int8_tensor_17x40x64": dict(A=A, B=B, A_scale=np.float32(sa), A_zero=np.int8(za),
                                        B_scale=np.float32(sb), B_zero=np.int8(zb), C=C, acc=acc)}
    M, N, K = 16, 24, 96
    A = g.integers(-127, 128, (M, K)).astype(np.int8)
    B = g.integers(-127, 128, (K, N)).astype(np.int8)
    sa = _f16(g.uniform(0.001, 0.02, M))
    sb = _f16(g.uniform(0.001, 0.02, N))
    C, acc = oracle.gemm_int8_rowcol(A, B, sa, sb)
    out["int8_rowcol_16x24x96"] = dict(A=A, B=B, sa=sa, sb=sb, C=C, acc=acc)
    return out


def int4_cases(g):
    out = {}
    M, N, K = 16, 5, 256
    G = K // 128
    qA = g.integers(0, 16, (M, K))
    qB = g.integers(0, 16, (K, N))
    # the reference's B layout [K, N/2] (gemm_int4.cu:49): odd N drops the last column
    A_q, B_q = quant.pack_rows(qA), quant.pack_cols(qB[:, :2 * (N // 2)])
    sA = _f16(g.uniform(0.001, 0.02, (M, G)))
    sB = _f16(g.uniform(0.001, 0.02, (G, N)))
    zA = _f16(g.integers(0, 16, (M, G)))
    zB = _f16(g.integers(0, 16, (G, N)))
    out["int4_literal_16x5x256"] = dict(
        A_q=A_q, A_scale=sA, A_zero=zA, B_q=B_q, B_scale=sB, B_zero=zB, M=np.int32(M),
        N=np.int32(N), K=np.int32(K), C=oracle.gemm_int4_literal(A_q, sA, B_q, sB, M, N, K))
    M, N, K = 16, 3, 384
    G = K // 128
    qA = g.integers(0, 16, (M, K))
    qB = g.integers(0, 16, (K, N))
    A_q, B_q = quant.pack_rows(qA), quant.pack_cols(qB)
    sA = _f16(g.uniform(0.001, 0.02, (M, G)))
    sB = _f16(g.uniform(0.001, 0.02, (G, N)))
    zA = _f16(g.integers(0, 16, (M, G)))
    zB = _f16(g.integers(0, 16, (G, N)))
    C, C64, part = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K, want_partials=True)
    out["int4_groupwise_16x3x384"] = dict(
        A_q=A_q, A_scale=sA, A_zero=zA, B_q=B_q, B_scale=sB, B_zero=zB, M=np.int32(M),
        N=np.int32(N), K=np.int32(K), C=C, C64=C64, partials=part)
    return out


def w4a16_cases(g):
    out = {}
    T, O, K = 3, 40, 256
    G = K // 128
    X = _f16(g.standard_normal((T, K)))
    W_q = quant.pack_rows(g.integers(0, 16, (O, K)))
    s = _f16(g.uniform(0.001, 0.02, (O, G)))
    z = _f16(g.integers(0, 16, (O, G)))
    Y_in = _f16(g.standard_normal((T, O)))
    Y, Y64 = oracle.w4a16(X, W_q, s, z, Y_in, 1.0, 1.0)
    out["w4a16_3x40x256_residual"] = dict(X=X, W_q=W_q, W_scale=s, W_zero=z, Y_in=Y_in,
                                          alpha=np.float32(1.0), beta=np.float32(1.0), Y=Y, Y64=Y64)
    T, I, K = 2, 24, 256
    G = K // 128
    X = _f16(g.standard_normal((T, K)))
    W_q = quant.pack_rows(g.integers(0, 16, (2 * I, K)))
    s = _f16(g.uniform(0.001, 0.02, (2 * I, G)))
    z = _f16(g.integers(0, 16, (2 * I, G)))
    out["w4a16_swiglu_2x24x256"] = dict(X=X, W_q=W_q, W_scale=s, W_zero=z, I=np.int32(I),
                                        H=oracle.w4a16_swiglu(X, W_q, s, z))
    gate = _f16(g.standard_normal(1000) * 4)
    up = _f16(g.standard_normal(1000))
    out["swiglu_1000"] = dict(gate=gate, up=up, out=oracle.swiglu(gate, up))
    return out


def main() -> None:
    g = np.random.default_rng(20261201)
    cases = {}
    for make in (fp16_cases, int8_cases, int4_cases, w4a16_cases):
        cases.update(make(g))
    for name, arrays in cases.items():
        np.savez(os.path.join(HERE, name + ".npz"), **arrays)
        print(name, ", ".join(f"{k}{list(np.shape(v))}" for k, v in arrays.items()))


if __name__ == "__main__":
    main()
