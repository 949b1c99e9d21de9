"""GPU parity of clove_gemm_fp16 / clove_gemm_fp16_batched against the oracle.

Shapes: the reference test's six cases (tests/test_gemm.cu:99-243), the
512^3 U[-1,1] workload and the LLM shapes with N(0,1) activations x N(0,0.02)
weights, ragged and unaligned shapes, and batched calls.  Bit-exact where the
mathematics fixes the answer (small-integer inputs); otherwise within
|got - ref| <= 1e-2 * max(|ref|, 1e-2 * rms(ref)) of the float64 oracle.
"""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, f16bits, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu


def _cg():
    import clove_compute_amd as cg
    return cg


def run_fp16(A, B, C0=None, alpha=1.0, beta=0.0):
    import torch
    M, K = A.shape
    N = B.shape[1]
    dA, dB = to_dev(A), to_dev(B)
    dC = to_dev(C0) if C0 is not None else empty_f16(M, N, fill=float("nan"))
    _cg().gemm_fp16(dA, dB, dC, M, N, K, alpha, beta)
    torch.cuda.synchronize()
    return to_host(dC)


def check_rows(A, B, C, rows, C0=None, alpha=1.0, beta=0.0):
    ref = oracle.gemm_fp16_f64(A[rows], B, None if C0 is None else C0[rows], alpha, beta)
    ok, rep = within_tol(C[rows], ref)
    assert ok, rep
    assert rep["ref_rule_failures"] == 0, rep


# the reference's own FP16 cases (tests/test_gemm.cu:99-219), inputs U[-0.1, 0.1)
@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (256, 256, 256), (1024, 1024, 1024),
                                   (128, 4096, 4096), (1, 4096, 4096)])
def test_reference_cases(M, N, K):
    g = rng("ref", M, N, K)
    A = g.uniform(-0.1, 0.1, (M, K)).astype(np.float16)
    B = g.uniform(-0.1, 0.1, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, min(M, 24))]))
    check_rows(A, B, C, rows)


def test_reference_alpha_beta():
    # tests/test_gemm.cu:221-243 (smoke-only there); checked here
    g = rng("alpha_beta")
    M = N = K = 128
    A = g.uniform(-0.1, 0.1, (M, K)).astype(np.float16)
    B = g.uniform(-0.1, 0.1, (K, N)).astype(np.float16)
    C0 = g.uniform(-0.1, 0.1, (M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=0.5, beta=0.25)
    check_rows(A, B, C, np.arange(M), C0, 0.5, 0.25)


def test_512_cubed_uniform_full():
    # 512^3, A and B ~ U[-1, 1]: every element against the oracle
    g = rng("cfg1")
    A = g.uniform(-1, 1, (512, 512)).astype(np.float16)
    B = g.uniform(-1, 1, (512, 512)).astype(np.float16)
    C = run_fp16(A, B)
    check_rows(A, B, C, np.arange(512))
    # the naive-arithmetic restatement agrees to a few fp16 ulps as well
    Co = oracle.gemm_fp16(A, B)
    assert np.max(np.abs(C.astype(np.float64) - Co.astype(np.float64))) < 4e-3 * 512 ** 0.5


@pytest.mark.parametrize("M", [1, 32, 128, 4096])
def test_llm_shapes(M):
    N = K = 4096
    g = rng("cfg2", M)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    C = run_fp16(A, B)
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, min(M, 16))]))
    check_rows(A, B, C, rows)
    assert np.all(np.isfinite(C.astype(np.float32)))


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (1, 4096, 4096), (7, 96, 300), (4096, 4096, 4096)])
def test_small_integer_inputs_bit_exact(M, N, K):
    # |a|,|b| <= 2: every fp32 partial sum is an exact integer, |C| < 2048 for
    # these sizes with overwhelming probability, so C is exact in any order
    g = rng("int", M, N, K)
    A = g.integers(-2, 3, (M, K)).astype(np.float16)
    B = g.integers(-2, 3, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))


@pytest.mark.parametrize("M,N,K", [(77, 45, 131), (3, 17, 33), (130, 257, 96), (33, 8, 8),
                                   (5, 4096, 64), (1, 7, 1), (300, 129, 1000)])
def test_ragged_and_unaligned(M, N, K):
    g = rng("ragged", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = g.standard_normal((K, N)).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=1.5, beta=-0.75)
    check_rows(A, B, C, np.arange(M), C0, 1.5, -0.75)


def test_k_zero_and_empty():
    import torch
    cg = _cg()
    C0 = np.arange(12, dtype=np.float16).reshape(3, 4)
    dC = to_dev(C0)
    dA = empty_f16(3, 1)
    dB = empty_f16(1, 4)
    cg.gemm_fp16(dA, dB, dC, 3, 4, 0, 1.0, 0.5)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(dC), (C0.astype(np.float32) * 0.5).astype(np.float16))
    cg.gemm_fp16(dA, dB, dC, 0, 4, 5)  # no-op
    cg.gemm_fp16(dA, dB, dC, 3, 0, 5)  # no-op


def test_beta_zero_ignores_nan_in_c():
    g = rng("nanc")
    A = g.integers(-3, 4, (64, 64)).astype(np.float16)
    B = g.integers(-3, 4, (64, 128)).astype(np.float16)
    C = run_fp16(A, B, np.full((64, 128), np.nan, np.float16), 1.0, 0.0)
    assert np.array_equal(f16bits(C), f16bits((A.astype(np.float64) @ B.astype(np.float64)).astype(np.float16)))


@pytest.mark.parametrize("batch,M,N,K", [(3, 64, 96, 80), (4, 1, 256, 512), (2, 300, 200, 64)])
def test_batched(batch, M, N, K):
    import torch
    g = rng("batched", batch, M, N, K)
    A = g.standard_normal((batch, M, K)).astype(np.float16)
    B = g.standard_normal((batch, K, N)).astype(np.float16)
    C0 = g.standard_normal((batch, M, N)).astype(np.float16)
    dC = to_dev(C0)
    _cg().gemm_fp16_batched(to_dev(A), to_dev(B), dC, batch, M, N, K, 0.5, 1.0)
    torch.cuda.synchronize()
    C = to_host(dC)
    for b in range(batch):
        ref = oracle.gemm_fp16_f64(A[b], B[b], C0[b], 0.5, 1.0)
        ok, rep = within_tol(C[b], ref)
        assert ok, (b, rep)


def test_repeat_calls_deterministic_split_k():
    # split-K shapes reduce in a fixed order: repeated calls are bit-identical
    import torch
    g = rng("det")
    M, N, K = 32, 4096, 4096
    A = to_dev(g.standard_normal((M, K)).astype(np.float16))
    B = to_dev((g.standard_normal((K, N)) * 0.02).astype(np.float16))
    outs = []
    for _ in range(3):
        C = empty_f16(M, N)
        _cg().gemm_fp16(A, B, C, M, N, K)
        torch.cuda.synchronize()
        outs.append(f16bits(to_host(C)))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


# ---- the 256x256x64 DMA-staged kernel (large, aligned shapes) ----

@pytest.mark.parametrize("M,N,K", [(2048, 4096, 512), (3000, 3000, 320), (4096, 2056, 128), (1536, 2048, 64)])
def test_big_tile_ragged_edges(M, N, K):
    # tile grids >= half the CUs with ragged M / N edges (rows past the end read
    # as zero, columns past N never stored); K / 64 odd (320) and 1 (64)
    g = rng("big", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.05).astype(np.float16)
    C = run_fp16(A, B)
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1], g.integers(0, M, 40)]))
    check_rows(A, B, C, rows)
    assert np.all(np.isfinite(C.astype(np.float32)))


def test_big_tile_every_element_small_integers():
    # every element bit-exact: small-integer inputs make any summation order exact
    M, N, K = 2304, 3840, 192
    g = rng("big_int")
    A = g.integers(-3, 4, (M, K)).astype(np.float16)
    B = g.integers(-3, 4, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))


def test_big_tile_alpha_beta():
    M = N = 3072
    K = 256
    g = rng("big_ab")
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.05).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=1.5, beta=-0.75)
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 24)]))
    check_rows(A, B, C, rows, C0, 1.5, -0.75)


def test_big_tile_batched():
    import torch
    batch, M, N, K = 2, 2048, 2048, 128
    g = rng("big_batched")
    A = g.standard_normal((batch, M, K)).astype(np.float16)
    B = (g.standard_normal((batch, K, N)) * 0.05).astype(np.float16)
    dC = empty_f16(batch, M, N, fill=float("nan"))
    _cg().gemm_fp16_batched(to_dev(A), to_dev(B), dC, batch, M, N, K, 1.0, 0.0)
    torch.cuda.synchronize()
    C = to_host(dC)
    for b in range(batch):
        rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 16)]))
        ref = oracle.gemm_fp16_f64(A[b][rows], B[b])
        ok, rep = within_tol(C[b][rows], ref)
        assert ok, (b, rep)


# the 256x256 kernel's K split: where its tiles cover only half the CUs (128
# tiles) and K >= 8192, each tile's K range in two parts, fp32 partials summed
# in split order by the last part (even and odd K-tile counts, ragged M and
# N); 128 tiles with shorter K and partly filled last rounds (344 and 288
# tiles) are not split
@pytest.mark.parametrize("M,N,K", [(2048, 4096, 8192), (1900, 4000, 8256), (2048, 4096, 1024), (2048, 11008, 1024),
                                   (1800, 9000, 1024)])
def test_big_tile_k_split_small_integers_bit_exact(M, N, K):
    g = rng("big_split_int", M, N, K)
    A = g.integers(-3, 4, (M, K)).astype(np.float16)
    B = g.integers(-3, 4, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))


@pytest.mark.parametrize("M,N,K,alpha,beta", [(2048, 4096, 11008, 1.0, 0.0), (1900, 4000, 8256, 0.5, 0.75)])
def test_big_tile_k_split(M, N, K, alpha, beta):
    g = rng("big_split", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16) if beta != 0.0 else None
    C = run_fp16(A, B, C0, alpha, beta)
    rows = np.unique(np.concatenate([[0, 255, 256, M - 256, M - 1], g.integers(0, M, 24)]))
    check_rows(A, B, C, rows, C0, alpha, beta)
    assert np.all(np.isfinite(C.astype(np.float32)))


def test_big_shape_k_not_multiple_of_tile():
    # K % 64 != 0 takes the generic MFMA kernel
    M, N, K = 4096, 4096, 1000
    g = rng("big_k1000")
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.05).astype(np.float16)
    C = run_fp16(A, B)
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 16)]))
    check_rows(A, B, C, rows)


# 4 < M <= 512 with K % 64 == 0, N % 8 == 0 and 16-byte aligned operands take
# the skinny kernel (B through LDS DMA and transposing LDS reads): every
# M configuration (<= 32, <= 64, <= 512), ragged M and N, split K, alpha/beta
@pytest.mark.parametrize("M,N,K", [(5, 4096, 4096), (17, 136, 192), (33, 520, 1024), (64, 4096, 2048),
                                   (65, 72, 64), (129, 1000, 4096), (250, 4096, 512), (512, 8, 128)])
def test_skinny_shapes(M, N, K):
    g = rng("skinny", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=0.75, beta=-0.5)
    rows = np.arange(M) if M <= 64 else np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 24)]))
    check_rows(A, B, C, rows, C0, 0.75, -0.5)


# short K with at most one 32x32 tile per CU: 32x32 tiles whose four waves
# each take one k-step of every K tile, the four sums added through LDS
# (alpha / beta, ragged M and N, M = 3 on a weight that skips the GEMV)
@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (64, 512, 1024), (3, 8192, 1024), (32, 4096, 512),
                                   (100, 200, 320)])
def test_k_sliced_small_tiles(M, N, K):
    g = rng("k-sliced", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=0.75, beta=-0.5)
    rows = np.arange(M) if M <= 100 else np.unique(np.concatenate([[0, 31, 32, M - 1], g.integers(0, M, 24)]))
    check_rows(A, B, C, rows, C0, 0.75, -0.5)


@pytest.mark.parametrize("M,N,K", [(7, 4096, 4096), (100, 264, 640), (128, 4096, 4096),
                                   (3, 4096, 4096), (2, 11008, 4096), (4, 4096, 11008),
                                   (512, 512, 1024), (3, 8192, 1024), (128, 4096, 11008)])
def test_skinny_small_integers_bit_exact(M, N, K):
    # |a|, |b| <= 4 integers: every product and partial sum is exact in fp32,
    # so split K and the fp16 output are exact (M = 2..4 on these weights
    # take the skinny kernel rather than the GEMV)
    g = rng("skinny-int", M, N, K)
    A = g.integers(-4, 5, (M, K)).astype(np.float16)
    B = g.integers(-4, 5, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    ref = oracle.gemm_fp16_f64(A, B).astype(np.float16)
    assert np.array_equal(f16bits(C), f16bits(ref))


# M = 1..4 on the GEMV with several K splits (K > 256), ragged last splits
# (8200, 11008, 4104) and a half column block (1032, 4104, 136): the per-row
# partials, split publication and reduce of every row count, beta != 0; small
# integers make every order exact, so the comparison is bit for bit
@pytest.mark.parametrize("M,N,K", [(2, 4096, 4096), (3, 1024, 2048), (4, 1024, 2048), (2, 1032, 8200),
                                   (1, 4104, 11008), (4, 136, 4104)])
def test_gemv_multirow_split_k_bit_exact(M, N, K):
    g = rng("gemv-mm", M, N, K)
    A = g.integers(-3, 4, (M, K)).astype(np.float16)
    B = g.integers(-3, 4, (K, N)).astype(np.float16)
    C0 = g.integers(-8, 9, (M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=1.0, beta=0.5)
    exact = A.astype(np.float64) @ B.astype(np.float64) + 0.5 * C0.astype(np.float64)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))


# M > 256 whose 256x256 tile grid would leave CUs idle: 128x128 tiles (with
# two K splits at 512x4096x4096) or 64x64 tiles (1024^3, and ragged edges)
@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (1024, 1024, 1024), (2048, 2048, 2048),
                                   (300, 1000, 640), (777, 520, 192)])
def test_mid_size_tiles(M, N, K):
    g = rng("mid", M, N, K)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.05).astype(np.float16)
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C = run_fp16(A, B, C0, alpha=0.5, beta=0.25)
    rows = np.unique(np.concatenate([[0, 63, 64, 127, 128, M - 1], g.integers(0, M, 24)]))
    check_rows(A, B, C, rows, C0, 0.5, 0.25)


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (1024, 1024, 1024), (600, 392, 320), (192, 11008, 4096),
                                   (384, 4096, 4096), (160, 1000, 2048), (128, 11008, 4096), (96, 10240, 4096)])
def test_mid_size_tiles_small_integers_bit_exact(M, N, K):
    g = rng("mid-int", M, N, K)
    A = g.integers(-2, 3, (M, K)).astype(np.float16)
    B = g.integers(-2, 3, (K, N)).astype(np.float16)
    C = run_fp16(A, B)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))
