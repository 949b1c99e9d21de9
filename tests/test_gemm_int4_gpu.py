"""GPU parity of clove_gemm_int4 / clove_gemm_int4_ex against the oracle.

Group-wise mode: within |got - ref| <= 1e-2 * max(|ref|, 1e-2 * rms(ref)) of
the float64 oracle, and bit-exact on power-of-two-scale cases where every
step is exact.  Reference-literal mode: bit-exact (integer sum, then the
reference's (acc * a_s) * b_s, src/kernels/gemm_int4.cu:185-190).
"""
import numpy as np
import pytest

import oracle
from clove_compute_amd import quant
from tests._util import empty_f16, f16bits, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu

LIT = 1


def _cg():
    import clove_compute_amd as cg
    return cg


def make_case(M, N, K, key, pow2=False, small=False):
    g = rng("i4", M, N, K, key)
    G = (K + 127) // 128
    if small:
        qA = g.integers(7, 10, (M, K))
        qB = g.integers(7, 10, (K, N))
    else:
        qA = g.integers(0, 16, (M, K))
        qB = g.integers(0, 16, (K, N))
    A_q = quant.pack_rows(qA)
    B_q = quant.pack_cols(qB)
    if pow2:
        sA = (2.0 ** -g.integers(0, 3, (M, G))).astype(np.float16)
        sB = (2.0 ** -g.integers(0, 3, (G, N))).astype(np.float16)
        zA = np.full((M, G), 8, np.float16)
        zB = np.full((G, N), 8, np.float16)
    else:
        sA = g.uniform(0.001, 0.02, (M, G)).astype(np.float16)
        sB = g.uniform(0.001, 0.02, (G, N)).astype(np.float16)
        zA = g.integers(0, 16, (M, G)).astype(np.float16)
        zB = g.integers(0, 16, (G, N)).astype(np.float16)
    return A_q, sA, zA, B_q, sB, zB


def run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K, mode=0):
    import torch
    C = empty_f16(M, N, fill=float("nan"))
    _cg().gemm_int4_ex(to_dev(A_q), to_dev(sA), None if zA is None else to_dev(zA),
                       None if B_q is None else to_dev(B_q), to_dev(sB),
                       None if zB is None else to_dev(zB), C, M, N, K, mode)
    torch.cuda.synchronize()
    return to_host(C)


@pytest.mark.parametrize("M,K", [(11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("N", [1, 16, 128])
def test_config4_groupwise(M, N, K):
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "cfg4")
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    g = rng("rows", M, N, K)
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 24)]))
    _, ref, _ = oracle.gemm_int4_groupwise(A_q[rows], sA[rows], zA[rows], B_q, sB, zB, len(rows), N, K)
    ok, rep = within_tol(C[rows], ref)
    assert ok, rep
    assert np.all(np.isfinite(C.astype(np.float32)))


# (N = 1 with K = 2080..4096 takes the GEMV whose two waves split K, with one,
# two or four rows per workgroup: 300, 1030 and 2050 rows, the last workgroup
# ragged; K = 2304 leaves lanes of the second wave without a chunk.  N = 16
# takes the raw-B streaming kernel with 48 rows per workgroup at 11000 rows
# and 32 at 8000, both ragged)
@pytest.mark.parametrize("M,N,K", [(300, 1, 4096), (260, 8, 2048), (100, 16, 1024), (130, 128, 512),
                                   (64, 3, 640), (1024, 4, 11008), (512, 8, 4096), (96, 6, 4104),
                                   (2050, 1, 4096), (1030, 1, 2304), (11000, 16, 4096), (8000, 16, 4096),
                                   (130, 1, 2080), (70, 1, 4128)])
def test_groupwise_pow2_bit_exact(M, N, K):
    # power-of-two scales, values q-z in [-1, 1]: every fp32/fp16 step is exact
    # (N = 1 on rows of 65..128 chunks of 32 k takes the two-wave K-split GEMV:
    # K = 2080 is its lower bound, the second wave holding one chunk, and K =
    # 4128 is just past its upper one)
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "pow2", pow2=True, small=True)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    Cr, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    assert np.array_equal(f16bits(C), f16bits(ref.astype(np.float16)))


@pytest.mark.parametrize("M,N,K", [(77, 5, 200), (33, 17, 96), (65, 40, 330), (9, 1, 64), (130, 7, 4096)])
def test_groupwise_ragged(M, N, K):
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "ragged")
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    _, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    ok, rep = within_tol(C, ref)
    assert ok, rep


@pytest.mark.parametrize("M,N,K", [(4096, 1, 11008), (11008, 16, 4096), (256, 128, 4096), (70, 7, 256),
                                   (40, 33, 320), (64, 2, 128)])
def test_literal_bit_exact(M, N, K):
    g = rng("lit", M, N, K)
    G = (K + 127) // 128
    qA = g.integers(0, 16, (M, K))
    A_q = quant.pack_rows(qA)
    sA = g.uniform(0.001, 0.02, (M, G)).astype(np.float16)
    sB = g.uniform(0.001, 0.02, (G, N)).astype(np.float16)
    hb = N // 2
    B_q = g.integers(0, 256, (K, hb)).astype(np.uint8) if hb > 0 else None
    C = run_int4(A_q, sA, None, B_q, sB, None, M, N, K, mode=LIT)
    rows = np.arange(M) if M <= 512 else np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 32)]))
    Bo = B_q if B_q is not None else np.zeros((K, 1), np.uint8)
    ref = oracle.gemm_int4_literal(A_q[rows], sA[rows], Bo, sB, len(rows), N, K)
    assert np.array_equal(f16bits(C[rows]), f16bits(ref))
    if N == 1:
        assert np.all(f16bits(C) == 0)


def test_quantizer_round_trip_through_kernel():
    # quantise real-valued weights/activations, multiply, compare with the
    # float64 product of the dequantised operands
    g = rng("quant")
    M, N, K = 256, 16, 1024
    W = g.standard_normal((M, K)) * 0.02
    X = g.standard_normal((K, N))
    A_q, sA, zA = quant.quantize_rows(W)
    B_q, sB, zB = quant.quantize_cols(X)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    ref = quant.dequantize_rows(A_q, sA, zA, K) @ quant.dequantize_rows(
        quant.pack_rows(quant.unpack_cols(B_q, N).T), sB.T, zB.T, K).T
    ok, rep = within_tol(C, ref)
    assert ok, rep


# group-wise, N > 8, K % 128 == 0 takes the INT4-weight MFMA kernel (i4w_gemm)
# after the B transpose: every tile configuration, ragged M and N (odd N: the
# last byte column's low nibble is padding), split K
@pytest.mark.parametrize("M,N,K", [(77, 17, 256), (300, 33, 1024), (129, 100, 512), (1000, 200, 1024),
                                   (8192, 1024, 256), (4096, 9, 11008)])
def test_groupwise_mfma_path(M, N, K):
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "mfma")
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    g = rng("rows-mfma", M, N, K)
    rows = np.arange(M) if M <= 1000 else np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 32)]))
    _, ref, _ = oracle.gemm_int4_groupwise(A_q[rows], sA[rows], zA[rows], B_q, sB, zB, len(rows), N, K)
    ok, rep = within_tol(C[rows], ref)
    assert ok, rep
    assert np.all(np.isfinite(C.astype(np.float32)))


@pytest.mark.parametrize("M,N,K", [(4096, 16, 11008), (1000, 200, 1024), (8192, 1024, 256)])
def test_groupwise_mfma_path_pow2_bit_exact(M, N, K):
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "pow2m", pow2=True, small=True)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    g = rng("rows-p2", M, N, K)
    rows = np.arange(M) if M <= 1000 else np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 32)]))
    _, ref, _ = oracle.gemm_int4_groupwise(A_q[rows], sA[rows], zA[rows], B_q, sB, zB, len(rows), N, K)
    assert np.array_equal(f16bits(C[rows]), f16bits(ref.astype(np.float16)))


# group-wise, 9..16 columns, K % 128 == 0: the streaming kernel
# (i4w_stream.hpp), after the B transpose for N < 15 and reading B in place
# for N = 15, 16: K slices of 2, 4 and 8 waves (G = 1, 2, 20, 40, 86), ragged
# M (fewer rows than one fragment), odd N (N = 15: the pad nibble of each B
# row is read and its column dropped)
@pytest.mark.parametrize("M,N,K", [(7, 9, 128), (5, 16, 128), (40, 16, 256), (300, 12, 2560), (1000, 16, 5120),
                                   (33, 15, 11008)])
def test_groupwise_stream_path(M, N, K):
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "stream")
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    _, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    ok, rep = within_tol(C, ref)
    assert ok, rep


def test_groupwise_stream_path_pow2_bit_exact():
    M, N, K = 520, 16, 4096
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "pow2st", pow2=True, small=True)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    _, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    assert np.array_equal(f16bits(C), f16bits(ref.astype(np.float16)))


# group-wise with N >= 64 and K % 256 == 0: the int8-MFMA kernel (i4i4_gemm)
# after the Bt pre-pass.  Zero points at both ends of its exact range
# [-112, 127] (q - z spans [-127, 127]) with power-of-two scales: every step
# exact, so bit for bit.
@pytest.mark.parametrize("M,N,K", [(130, 64, 512), (257, 136, 1024), (1, 64, 256)])
def test_int8_mfma_path_zero_point_range_bit_exact(M, N, K):
    g = rng("i4i4-range", M, N, K)
    G = K // 128
    A_q = quant.pack_rows(g.integers(0, 16, (M, K)))
    B_q = quant.pack_cols(g.integers(0, 16, (K, N)))
    ends = np.array([-112, 127, 0, 15, 8], np.float16)
    zA = ends[g.integers(0, 5, (M, G))]
    zB = ends[g.integers(0, 5, (G, N))]
    # one power of two for every scale: |C| < 2^8 in steps of 2^-16, so the
    # fp32 sums are exact and the fp16 results finite
    sA = np.full((M, G), 2.0 ** -8, np.float16)
    sB = np.full((G, N), 2.0 ** -8, np.float16)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    _, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    assert np.array_equal(f16bits(C), f16bits(ref.astype(np.float16)))


@pytest.mark.parametrize("M,K", [(4096, 11008), (11008, 4096)])
def test_int8_mfma_path_config4_n128_every_row_bit_exact(M, K):
    # the config-4 prefill shapes on the int8-MFMA kernel, every row and
    # column: power-of-two scales and q - z in [-1, 1], so every per-group
    # sum, scale product and fp32 fold is exact and the output is the fp16
    # rounding of the exact value (computed here in float64, group by group)
    N = 128
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "pow2-cfg4", pow2=True, small=True)
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    G = K // 128
    a = quant.unpack_rows(A_q, K).astype(np.float64).reshape(M, G, 128) - zA.astype(np.float64)[:, :, None]
    b = quant.unpack_cols(B_q, N).astype(np.float64).reshape(G, 128, N) - zB.astype(np.float64)[:, None, :]
    ref = np.zeros((M, N))
    for g in range(G):
        ref += sA[:, g, None].astype(np.float64) * sB[None, g, :].astype(np.float64) * (a[:, g, :] @ b[g])
    assert np.array_equal(f16bits(C), f16bits(ref.astype(np.float16)))


def test_int8_mfma_path_zero_point_outside_range_is_nan():
    # a zero point the int8 operands cannot hold exactly poisons exactly the
    # outputs whose sum it enters (its row, or its column), nothing else
    M, N, K = 192, 128, 512
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "nan")
    zA[5, 2] = 200.0
    zB[1, 77] = -120.0
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    bad = np.zeros((M, N), bool)
    bad[5, :] = True
    bad[:, 77] = True
    assert np.all(np.isnan(C[bad].astype(np.float32)))
    _, ref, _ = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K)
    ok, rep = within_tol(C[~bad], ref[~bad])
    assert ok, rep


@pytest.mark.parametrize("M,N,K", [(4096, 128, 11008), (600, 100, 2816), (1000, 320, 1024),
                                   (11008, 128, 4096), (8192, 512, 512)])
def test_int8_mfma_path_split_k(M, N, K):
    # 64-row tiles split over groups (G = 86 in four splits of 22, 22, 22 and
    # 20 groups; G = 22 in eleven splits of two), N not a multiple of 8
    # (element stores), two and three column tiles, 64-row tiles without a
    # split (11008 rows) and 128-row tiles (8192 x 512: 256 tiles)
    A_q, sA, zA, B_q, sB, zB = make_case(M, N, K, "i4i4-split")
    C = run_int4(A_q, sA, zA, B_q, sB, zB, M, N, K)
    g = rng("rows-i4i4", M, N, K)
    rows = np.arange(M) if M <= 1000 else np.unique(np.concatenate([[0, 127, 128, M - 1], g.integers(0, M, 32)]))
    _, ref, _ = oracle.gemm_int4_groupwise(A_q[rows], sA[rows], zA[rows], B_q, sB, zB, len(rows), N, K)
    ok, rep = within_tol(C[rows], ref)
    assert ok, rep


def run_group_acc32(A_q, zA, B_q, zB, M, N, K):
    import torch
    G = K // 128
    P = torch.full((M, N, G), 12345, dtype=torch.int32, device="cuda")
    _cg().gemm_int4_group_acc32(to_dev(A_q), to_dev(zA), to_dev(B_q), to_dev(zB), P, M, N, K)
    torch.cuda.synchronize()
    return P.cpu().numpy()


def partials_int64(A_q, zA, B_q, zB, rows, N, K):
    # independent restatement: unpack with numpy, int64 sums per group
    qA = quant.unpack_rows(A_q[rows], K).astype(np.int64)           # [r, K]
    qB = quant.unpack_cols(B_q, N).astype(np.int64)                 # [K, N]
    G = K // 128
    za = np.rint(zA[rows].astype(np.float64)).astype(np.int64)     # [r, G]
    zb = np.rint(zB.astype(np.float64)).astype(np.int64)           # [G, N]
    a = (qA.reshape(len(rows), G, 128) - za[:, :, None])           # [r, G, 128]
    b = (qB.reshape(G, 128, N) - zb[:, None, :])                   # [G, 128, N]
    return np.einsum("rgk,gkn->rng", a, b)


# The int8-MFMA kernel's per-group integer sums P_g, through the partials hook
# (its LDS DMAs carry their own wait states: without them the compiled hook
# read weight rows as zeros after restoring a spilled resource SGPR, see
# tests/test_hazards.py):
# bit for bit against the oracle's partials and an independent numpy int64
# restatement, with arbitrary zero points over the kernel's whole exact range
# [-112, 127] (not only 8) and ragged M / N.
@pytest.mark.parametrize("M,N,K", [(130, 64, 512), (64, 1, 256), (257, 200, 1024), (1000, 128, 11008)])
def test_group_partials_bit_exact(M, N, K):
    g = rng("i4-partials", M, N, K)
    G = K // 128
    A_q = quant.pack_rows(g.integers(0, 16, (M, K)))
    B_q = quant.pack_cols(g.integers(0, 16, (K, N)))
    zA = g.integers(-112, 128, (M, G)).astype(np.float16)
    zB = g.integers(-112, 128, (G, N)).astype(np.float16)
    P = run_group_acc32(A_q, zA, B_q, zB, M, N, K)
    rows = np.arange(M) if M <= 300 else np.unique(np.concatenate([[0, 63, 64, M - 1], g.integers(0, M, 24)]))
    ref = partials_int64(A_q, zA, B_q, zB, rows, N, K)
    assert np.array_equal(P[rows].astype(np.int64), ref)
    if M <= 300:
        sA = np.ones((M, G), np.float16)
        sB = np.ones((G, N), np.float16)
        _, _, part = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K, want_partials=True)
        assert np.array_equal(P, part)


def test_group_partials_zero_point_outside_range():
    # a zero point the int8 operands cannot hold marks exactly the partials of
    # its row (or column) and group with INT32_MIN
    M, N, K = 70, 90, 512
    g = rng("i4-partials-bad", M, N, K)
    G = K // 128
    A_q = quant.pack_rows(g.integers(0, 16, (M, K)))
    B_q = quant.pack_cols(g.integers(0, 16, (K, N)))
    zA = g.integers(0, 16, (M, G)).astype(np.float16)
    zB = g.integers(0, 16, (G, N)).astype(np.float16)
    zA[3, 1] = 130.0
    zB[2, 40] = -113.0
    P = run_group_acc32(A_q, zA, B_q, zB, M, N, K)
    bad = np.zeros((M, N, G), bool)
    bad[3, :, 1] = True
    bad[:, 40, 2] = True
    assert np.all(P[bad] == np.iinfo(np.int32).min)
    ref = partials_int64(A_q, zA, B_q, zB, np.arange(M), N, K)
    assert np.array_equal(P[~bad].astype(np.int64), ref[~bad])
