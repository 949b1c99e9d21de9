"""GPU parity of the INT8 entry points against the oracle: bit-exact.

int32 accumulators are compared through clove_gemm_int8_acc32 (the same
kernels with an integer epilogue) and the fp16 outputs are compared bit for
bit: C = fp16(float(acc) * scale) has exactly one well-defined rounding chain.
"""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, f16bits, rng, to_dev, to_host

pytestmark = pytest.mark.gpu


def _cg():
    import clove_compute_amd as cg
    return cg


def _sync():
    import torch
    torch.cuda.synchronize()


def run_acc32(A, B, za=0, zb=0):
    import torch
    M, K = A.shape
    N = B.shape[1]
    acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
    _cg().gemm_int8_acc32(to_dev(A), to_dev(B), acc, M, N, K, za, zb)
    _sync()
    return acc.cpu().numpy()


@pytest.mark.parametrize("M", [1, 128])
def test_config3_w8a8_rowcol(M):
    # weights int8 U[-127,127] with per-channel fp16 scales, activations int8
    # with per-token fp16 scales, zero points 0
    N = K = 4096
    g = rng("cfg3", M)
    A = g.integers(-127, 128, (M, K)).astype(np.int8)
    B = g.integers(-127, 128, (K, N)).astype(np.int8)
    sa = g.uniform(0.001, 0.02, M).astype(np.float16)
    sb = g.uniform(0.001, 0.02, N).astype(np.float16)
    C = empty_f16(M, N)
    _cg().gemm_int8_rowcol(to_dev(A), to_dev(B), to_dev(sa), to_dev(sb), C, M, N, K)
    _sync()
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, min(M, 16))]))
    Cref, accref = oracle.gemm_int8_rowcol(A[rows], B, sa[rows], sb)
    assert np.array_equal(f16bits(to_host(C)[rows]), f16bits(Cref))
    acc = run_acc32(A, B)
    assert np.array_equal(acc[rows], accref)
    # every accumulator at full size: float64 BLAS on integers is exact here
    full = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(acc.astype(np.float64), full)


@pytest.mark.parametrize("M,N,K,za,zb", [
    (1, 4096, 4096, 0, 0), (1, 512, 1000, 3, -5), (3, 256, 256, -128, 127), (4, 96, 64, 7, 7),
    (64, 64, 64, 0, 0), (200, 130, 300, 5, -9), (129, 4096, 512, -3, 2), (37, 19, 45, 1, 1),
    (512, 512, 512, 0, 0), (1000, 1024, 1024, 0, 0), (2048, 256, 2048, 0, 0), (96, 11008, 4096, 0, 0),
    (128, 11008, 4096, 0, 0), (100, 10240, 4096, 0, 0),
])
def test_per_tensor_bit_exact(M, N, K, za, zb):
    g = rng("pt", M, N, K, za, zb)
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    sa, sb = np.float32(g.uniform(0.001, 0.05)), np.float32(g.uniform(0.001, 0.05))
    C = empty_f16(M, N)
    _cg().gemm_int8(to_dev(A), to_dev(B), C, M, N, K, float(sa), za, float(sb), zb)
    _sync()
    Cref, accref = oracle.gemm_int8(A, B, sa, za, sb, zb)
    assert np.array_equal(f16bits(to_host(C)), f16bits(Cref))
    assert np.array_equal(run_acc32(A, B, za, zb), accref)


# The reference kernel's own accumulator at ragged K (CLOVE_INT8_REFERENCE_LITERAL):
# each zero-padded k of its last 32-wide K tile adds A_zero * B_zero
# (src/kernels/gemm_int8.cu:52-54, 63-64, 89-93).  Bit for bit against the
# oracle's restatement of that tile loop, on the GEMV (M <= 4) and MFMA routes;
# with K % 32 == 0 or a zero point 0 the mode equals the exact one.
@pytest.mark.parametrize("M,N,K,za,zb", [
    (1, 512, 1000, 3, -5), (200, 130, 300, 5, -9), (37, 19, 45, 1, 1), (4, 96, 70, 7, 7),
    (129, 4096, 520, -3, 2), (64, 64, 64, 4, 4), (33, 40, 100, 0, 9),
])
def test_reference_literal_mode_bit_exact(M, N, K, za, zb):
    g = rng("lit8", M, N, K, za, zb)
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    sa, sb = np.float32(g.uniform(0.001, 0.05)), np.float32(g.uniform(0.001, 0.05))
    cg = _cg()
    C = empty_f16(M, N)
    cg.gemm_int8_ex(to_dev(A), to_dev(B), C, M, N, K, float(sa), za, float(sb), zb,
                    cg.CLOVE_INT8_REFERENCE_LITERAL)
    Ce = empty_f16(M, N)
    cg.gemm_int8_ex(to_dev(A), to_dev(B), Ce, M, N, K, float(sa), za, float(sb), zb, cg.CLOVE_INT8_EXACT)
    _sync()
    Clit, _ = oracle.gemm_int8_literal(A, B, sa, za, sb, zb)
    Cex, _ = oracle.gemm_int8(A, B, sa, za, sb, zb)
    assert np.array_equal(f16bits(to_host(C)), f16bits(Clit))
    assert np.array_equal(f16bits(to_host(Ce)), f16bits(Cex))
    if (32 * ((K + 31) // 32) - K) * za * zb == 0:
        assert np.array_equal(f16bits(Clit), f16bits(Cex))


def test_reference_race_region_is_correct():
    # the reference kernel's 64x64 tiles let threads write outside their tile
    # (src/kernels/gemm_int8.cu:29-34 vs :9-10); every element here must equal
    # the per-element formula, including far from the first tile
    g = rng("race")
    M, N, K = 192, 320, 96
    A = g.integers(-50, 50, (M, K)).astype(np.int8)
    B = g.integers(-50, 50, (K, N)).astype(np.int8)
    C = empty_f16(M, N)
    _cg().gemm_int8(to_dev(A), to_dev(B), C, M, N, K, 0.01, 0, 0.02, 0)
    _sync()
    Cref, _ = oracle.gemm_int8(A, B, np.float32(0.01), 0, np.float32(0.02), 0)
    assert np.array_equal(f16bits(to_host(C)), f16bits(Cref))


def test_broadcast_rowcol_equals_per_tensor():
    g = rng("bcast")
    M, N, K = 64, 256, 512
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    s1, s2 = np.float16(0.0137), np.float16(0.0061)
    C1, C2 = empty_f16(M, N), empty_f16(M, N)
    _cg().gemm_int8(to_dev(A), to_dev(B), C1, M, N, K, float(s1), 2, float(s2), -3)
    _cg().gemm_int8_rowcol(to_dev(A), to_dev(B), to_dev(np.full(M, s1)), to_dev(np.full(N, s2)), C2,
                           M, N, K, 2, -3)
    _sync()
    assert np.array_equal(f16bits(to_host(C1)), f16bits(to_host(C2)))


# 4 < M <= 512, zero points 0, K % 128 == 0, N % 16 == 0: the skinny kernel
# (int8 B through LDS DMA and ds_read_b64_tr_b8); int32 partials keep split K exact
@pytest.mark.parametrize("M,N,K", [(5, 4096, 4096), (31, 272, 384), (64, 1024, 4096), (100, 48, 128),
                                   (128, 4096, 1024), (300, 512, 2048)])
def test_skinny_bit_exact(M, N, K):
    g = rng("skinny8", M, N, K)
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    sa = g.uniform(0.001, 0.02, M).astype(np.float16)
    sb = g.uniform(0.001, 0.02, N).astype(np.float16)
    s1, s2 = np.float32(g.uniform(0.001, 0.05)), np.float32(g.uniform(0.001, 0.05))
    C1, C2 = empty_f16(M, N), empty_f16(M, N)
    _cg().gemm_int8(to_dev(A), to_dev(B), C1, M, N, K, float(s1), 0, float(s2), 0)
    _cg().gemm_int8_rowcol(to_dev(A), to_dev(B), to_dev(sa), to_dev(sb), C2, M, N, K)
    _sync()
    Cref1, accref = oracle.gemm_int8(A, B, s1, 0, s2, 0)
    Cref2, _ = oracle.gemm_int8_rowcol(A, B, sa, sb)
    assert np.array_equal(run_acc32(A, B), accref)
    assert np.array_equal(f16bits(to_host(C1)), f16bits(Cref1))
    assert np.array_equal(f16bits(to_host(C2)), f16bits(Cref2))


# M = 2..4 on the GEMV with several K splits, non-zero zero points: per-tensor,
# row/column scales and the raw accumulators, each bit for bit
@pytest.mark.parametrize("M,N,K,za,zb", [(2, 4096, 4096, 3, -5), (3, 512, 2048, -7, 11), (4, 512, 2048, 9, -2),
                                         (4, 4096, 4096, 0, 0), (3, 11008, 4096, 0, 0), (4, 4096, 11008, 0, 0),
                                         (4, 11008, 4096, 3, -5)])
def test_gemv_multirow_split_k(M, N, K, za, zb):
    # (3 and 4 rows on 11008-wide weights take the skinny kernel when the zero
    # points are 0, the GEMV otherwise)
    g = rng("gemv8-mm", M, N, K, za, zb)
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    sa = g.uniform(0.001, 0.02, M).astype(np.float16)
    sb = g.uniform(0.001, 0.02, N).astype(np.float16)
    s1, s2 = np.float32(g.uniform(0.001, 0.05)), np.float32(g.uniform(0.001, 0.05))
    C1, C2 = empty_f16(M, N), empty_f16(M, N)
    _cg().gemm_int8(to_dev(A), to_dev(B), C1, M, N, K, float(s1), za, float(s2), zb)
    _cg().gemm_int8_rowcol(to_dev(A), to_dev(B), to_dev(sa), to_dev(sb), C2, M, N, K, za, zb)
    _sync()
    Cref1, accref = oracle.gemm_int8(A, B, s1, za, s2, zb)
    Cref2, _ = oracle.gemm_int8_rowcol(A, B, sa, sb, za, zb)
    assert np.array_equal(run_acc32(A, B, za, zb), accref)
    assert np.array_equal(f16bits(to_host(C1)), f16bits(Cref1))
    assert np.array_equal(f16bits(to_host(C2)), f16bits(Cref2))


# 256x256 tiles covering half the CUs: the LDS-DMA kernel (i8_dma_gemm.hpp);
# ragged M and N edges, K / 128 odd and 2; per-tensor, row / column scales
# and the raw accumulators, bit for bit on sampled rows
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (4100, 2000, 256), (2304, 3968, 640), (768, 11008, 512)])
def test_big_tile(M, N, K):
    import torch
    g = rng("i8big", M, N, K)
    A = g.integers(-128, 128, (M, K)).astype(np.int8)
    B = g.integers(-128, 128, (K, N)).astype(np.int8)
    sa = g.uniform(0.001, 0.02, M).astype(np.float16)
    sb = g.uniform(0.001, 0.02, N).astype(np.float16)
    s1, s2 = np.float32(g.uniform(0.001, 0.05)), np.float32(g.uniform(0.001, 0.05))
    dA, dB = to_dev(A), to_dev(B)
    C1, C2 = empty_f16(M, N), empty_f16(M, N)
    acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
    cg = _cg()
    cg.gemm_int8(dA, dB, C1, M, N, K, float(s1), 0, float(s2), 0)
    cg.gemm_int8_rowcol(dA, dB, to_dev(sa), to_dev(sb), C2, M, N, K)
    cg.gemm_int8_acc32(dA, dB, acc, M, N, K, 0, 0)
    _sync()
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1], g.integers(0, M, 24)]))
    Cref1, accref = oracle.gemm_int8(A[rows], B, s1, 0, s2, 0)
    Cref2, _ = oracle.gemm_int8_rowcol(A[rows], B, sa[rows], sb)
    assert np.array_equal(acc.cpu().numpy()[rows], accref)
    assert np.array_equal(f16bits(to_host(C1)[rows]), f16bits(Cref1))
    assert np.array_equal(f16bits(to_host(C2)[rows]), f16bits(Cref2))
