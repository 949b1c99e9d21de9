"""Pins the CPU oracle before anything is checked against it.

Each check is independent of the oracle's own loops: numpy's IEEE conversions,
numpy integer/float64 matmuls, exact small-integer cases, identity and K=1
closed forms.  A plausible oracle mistake (dropped term, swapped nibble,
transposed operand, wrong group, wrong rounding) fails at least one of them.
Runs on the CPU only.
"""
import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(20261201)


def f16bits(a):
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def ordered(a):
    """fp16 values -> integers whose differences count ulps (+0 and -0 coincide)."""
    b = f16bits(a).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


# ---------------------------------------------------------------------------
# binary16 conversions
# ---------------------------------------------------------------------------
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = oracle.f16_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    edge = np.array([
        0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e30, -1e30,
        np.inf, -np.inf, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
        2.0 ** -24 * 1.5, 2.0 ** -24 * 2.5, 2.0 ** -26, 1e-45,
        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2048.0 + 1.0, 2048.0 + 3.0,
        0.1, 1.0 / 3.0, 6.1e-5, 6.0e-5,
    ], dtype=np.float32)
    # every f16 value, every midpoint between neighbours, and random floats
    h = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16)
    vals = h.view(np.float16).astype(np.float32)
    mids = ((vals[:-1].astype(np.float64) + vals[1:].astype(np.float64)) / 2).astype(np.float32)
    rand = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 100.0, 3e4)
    ])
    x = np.concatenate([edge, vals, mids, -mids, rand])
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    nan = oracle.f32_to_f16(np.array([np.nan], np.float32)).view(np.float16)
    assert np.isnan(nan[0])


# ---------------------------------------------------------------------------
# FP16 GEMM
# ---------------------------------------------------------------------------
def test_fp16_small_integers_bit_exact():
    # integers |a|,|b| <= 8 with K=256: every fp32 partial sum is exact, so C is
    # the RNE rounding of the exact integer product in any summation order
    M, N, K = 37, 53, 256
    A = RNG.integers(-8, 9, (M, K)).astype(np.float16)
    B = RNG.integers(-8, 9, (K, N)).astype(np.float16)
    exact = A.astype(np.int64) @ B.astype(np.int64)
    C = oracle.gemm_fp16(A, B)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float64).astype(np.float16)))


def test_fp16_alpha_beta_closed_form():
    M, N, K = 16, 24, 64
    A = RNG.integers(-4, 5, (M, K)).astype(np.float16)
    B = RNG.integers(-4, 5, (K, N)).astype(np.float16)
    C0 = RNG.integers(-64, 65, (M, N)).astype(np.float16)
    exact = 0.5 * (A.astype(np.int64) @ B.astype(np.int64)) + 0.25 * C0.astype(np.float64)
    C = oracle.gemm_fp16(A, B, C0, alpha=0.5, beta=0.25)
    assert np.array_equal(f16bits(C), f16bits(exact.astype(np.float16)))
    # beta = 0 ignores C entirely (even NaN in C)
    Cn = np.full((M, N), np.nan, np.float16)
    C2 = oracle.gemm_fp16(A, B, Cn, alpha=1.0, beta=0.0)
    assert np.array_equal(f16bits(C2), f16bits((A.astype(np.int64) @ B.astype(np.int64)).astype(np.float16)))


def test_fp16_identity_and_k1():
    A = RNG.standard_normal((29, 64)).astype(np.float16)
    C = oracle.gemm_fp16(A, np.eye(64, dtype=np.float16))
    assert np.array_equal(f16bits(C), f16bits(A))
    a = RNG.standard_normal((33, 1)).astype(np.float16)
    b = RNG.standard_normal((1, 17)).astype(np.float16)
    C = oracle.gemm_fp16(a, b)
    ref = (a.astype(np.float32) * b.astype(np.float32)).astype(np.float16)  # exact product, one rounding
    assert np.array_equal(f16bits(C), f16bits(ref))


@pytest.mark.parametrize("M,N,K", [(1, 64, 4096), (31, 47, 515), (64, 64, 64)])
def test_fp16_random_forward_error_bound(M, N, K):
    A = RNG.standard_normal((M, K)).astype(np.float16)
    B = (RNG.standard_normal((K, N)) * 0.02).astype(np.float16)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    C = oracle.gemm_fp16(A, B).astype(np.float64)
    absprod = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    bound = K * 2.0 ** -24 * absprod * 1.01 + 2.0 ** -11 * np.abs(ref) + 2.0 ** -25
    assert np.all(np.abs(C - ref) <= bound)
    # the float64 closed form agrees with numpy to rounding
    f64 = oracle.gemm_fp16_f64(A, B)
    assert np.allclose(f64, ref, rtol=1e-12, atol=1e-12)


def test_fp16_transposed_operand_is_caught():
    # a square product where A@B != B@A: the oracle must match the former
    A = RNG.integers(-3, 4, (16, 16)).astype(np.float16)
    B = RNG.integers(-3, 4, (16, 16)).astype(np.float16)
    C = oracle.gemm_fp16(A, B).astype(np.int64)
    assert np.array_equal(C, A.astype(np.int64) @ B.astype(np.int64))
    assert not np.array_equal(C, B.astype(np.int64) @ A.astype(np.int64))


def test_fp16_row_range_only_touches_rows():
    A = RNG.integers(-3, 4, (8, 32)).astype(np.float16)
    B = RNG.integers(-3, 4, (32, 8)).astype(np.float16)
    C0 = np.full((8, 8), 7.0, np.float16)
    C = oracle.gemm_fp16(A, B, C0, rows=(2, 5))
    full = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float16)
    assert np.array_equal(C[2:5], full[2:5])
    assert np.all(C[:2] == 7.0) and np.all(C[5:] == 7.0)


@pytest.mark.parametrize("nthreads", [1, 3, 8])
def test_fp16_threaded_rows_equal_single_thread(nthreads):
    # the all-cores CPU baseline: rows spread over threads, same bits as one
    # thread (random fp16 operands, so the order of every sum matters), rows
    # outside the range untouched
    A = RNG.standard_normal((13, 96)).astype(np.float16)
    B = RNG.standard_normal((96, 40)).astype(np.float16)
    C0 = RNG.standard_normal((13, 40)).astype(np.float16)
    ref = oracle.gemm_fp16(A, B, C0, alpha=0.5, beta=0.25, rows=(2, 11))
    got = oracle.gemm_fp16_mt(A, B, (2, 11), nthreads, C0, alpha=0.5, beta=0.25)
    assert np.array_equal(f16bits(got), f16bits(ref))
    assert np.array_equal(f16bits(got[:2]), f16bits(C0[:2]))
    assert np.array_equal(f16bits(got[11:]), f16bits(C0[11:]))
    # and against the float64 closed form within the forward-error bound
    f64 = oracle.gemm_fp16_f64(A[2:11], B, C0[2:11], 0.5, 0.25)
    assert np.all(np.abs(got[2:11].astype(np.float64) - f64) <= 1e-2 * np.maximum(np.abs(f64), 1e-1))


def test_fp16_batched_matches_per_batch():
    A = RNG.integers(-4, 5, (3, 10, 20)).astype(np.float16)
    B = RNG.integers(-4, 5, (3, 20, 12)).astype(np.float16)
    C = oracle.gemm_fp16_batched(A, B, alpha=2.0)
    for b in range(3):
        ref = 2.0 * (A[b].astype(np.int64) @ B[b].astype(np.int64))
        assert np.array_equal(f16bits(C[b]), f16bits(ref.astype(np.float16)))


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("za,zb", [(0, 0), (3, -5), (-128, 127)])
def test_int8_accumulators_and_epilogue(za, zb):
    M, N, K = 19, 45, 300
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    sa, sb = np.float32(0.0123), np.float32(0.0071)
    C, acc = oracle.gemm_int8(A, B, sa, za, sb, zb)
    ref = (A.astype(np.int64) - za) @ (B.astype(np.int64) - zb)
    assert np.array_equal(acc.astype(np.int64), ref)
    cs = np.float32(sa * sb)
    assert np.array_equal(f16bits(C), f16bits((ref.astype(np.float32) * cs).astype(np.float16)))


def test_int8_rowcol_and_per_tensor_agree():
    M, N, K = 7, 33, 129
    A = RNG.integers(-127, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-127, 128, (K, N)).astype(np.int8)
    sa = RNG.uniform(0.001, 0.02, M).astype(np.float16)
    sb = RNG.uniform(0.001, 0.02, N).astype(np.float16)
    C, acc = oracle.gemm_int8_rowcol(A, B, sa, sb, 2, -1)
    ref = (A.astype(np.int64) - 2) @ (B.astype(np.int64) + 1)
    assert np.array_equal(acc.astype(np.int64), ref)
    cs = sa.astype(np.float32)[:, None] * sb.astype(np.float32)[None, :]
    assert np.array_equal(f16bits(C), f16bits((ref.astype(np.float32) * cs).astype(np.float16)))
    # broadcast scales reproduce the per-tensor call bit for bit
    s1, s2 = np.float16(0.0156), np.float16(0.0039)
    Cr, _ = oracle.gemm_int8_rowcol(A, B, np.full(M, s1), np.full(N, s2), 2, -1)
    Ct, _ = oracle.gemm_int8(A, B, np.float32(s1), 2, np.float32(s2), -1)
    assert np.array_equal(f16bits(Cr), f16bits(Ct))


@pytest.mark.parametrize("M,N,K,za,zb", [(37, 19, 45, 1, 1), (1, 512, 1000, 3, -5), (200, 130, 300, 5, -9),
                                          (9, 7, 64, 4, 3), (5, 6, 33, 0, 7), (5, 6, 33, -8, 0)])
def test_int8_reference_literal(M, N, K, za, zb):
    # the reference kernel at ragged K: each of the 32 * ceil(K / 32) - K
    # zero-padded k of its last 32-wide tile adds (0 - za)(0 - zb) to the
    # accumulator (src/kernels/gemm_int8.cu:52-54, 63-64, 89-93); pinned against
    # the exact sum plus that closed-form term, numpy int64
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    sa, sb = np.float32(0.0123), np.float32(0.0071)
    Cl, accl = oracle.gemm_int8_literal(A, B, sa, za, sb, zb)
    Ce, acce = oracle.gemm_int8(A, B, sa, za, sb, zb)
    exact = (A.astype(np.int64) - za) @ (B.astype(np.int64) - zb)
    pad = 32 * ((K + 31) // 32) - K
    assert np.array_equal(acce.astype(np.int64), exact)
    assert np.array_equal(accl.astype(np.int64), exact + pad * za * zb)
    cs = np.float32(sa * sb)
    lit = ((exact + pad * za * zb).astype(np.float32) * cs).astype(np.float16)
    assert np.array_equal(f16bits(Cl), f16bits(lit))
    if pad * za * zb == 0:  # K % 32 == 0 or a zero point 0: the two agree
        assert np.array_equal(f16bits(Cl), f16bits(Ce))
    else:
        assert np.all(accl.astype(np.int64) - acce.astype(np.int64) == pad * za * zb)


def test_int8_reference_literal_difference_at_37x19x45():
    # K = 45: the last tile holds 19 padded k, so with zero points (1, 1) the
    # reference's accumulator is the exact sum + 19
    A = RNG.integers(-128, 128, (37, 45)).astype(np.int8)
    B = RNG.integers(-128, 128, (45, 19)).astype(np.int8)
    _, accl = oracle.gemm_int8_literal(A, B, 1.0, 1, 1.0, 1)
    _, acce = oracle.gemm_int8(A, B, 1.0, 1, 1.0, 1)
    assert np.all(accl.astype(np.int64) - acce == 19)


# ---------------------------------------------------------------------------
# INT4
# ---------------------------------------------------------------------------
def pack_rows(q):
    """[R, K] nibbles -> [R, K/2] bytes, even k in the high nibble."""
    q = q.astype(np.uint8)
    return ((q[:, 0::2] << 4) | q[:, 1::2]).astype(np.uint8)


def pack_cols(q, stride):
    """[K, N] nibbles -> [K, stride] bytes, even n in the high nibble."""
    K, N = q.shape
    out = np.zeros((K, stride), np.uint8)
    for j in range(stride):
        hi = q[:, 2 * j] if 2 * j < N else 0
        lo = q[:, 2 * j + 1] if 2 * j + 1 < N else 0
        out[:, j] = (np.asarray(hi, np.uint8) << 4) | np.asarray(lo, np.uint8)
    return out


@pytest.mark.parametrize("M,N,K", [(9, 16, 256), (5, 7, 384), (4, 1, 128), (3, 10, 320)])
def test_int4_literal(M, N, K):
    G = (K + 127) // 128
    qA = RNG.integers(0, 16, (M, K))
    qB = RNG.integers(0, 16, (K, N))
    sA = RNG.uniform(0.001, 0.02, (M, G)).astype(np.float16)
    sB = RNG.uniform(0.001, 0.02, (G, N)).astype(np.float16)
    A_q = pack_rows(qA)
    B_q = pack_cols(qB, N // 2) if N >= 2 else np.zeros((K, 1), np.uint8)
    C = oracle.gemm_int4_literal(A_q, sA, B_q, sB, M, N, K)
    vB = (qB - 8).astype(np.int64)
    vB[:, 2 * (N // 2):] = 0             # the reference never loads these columns
    S = (qA - 8).astype(np.int64) @ vB
    a_s = sA[:, G - 1].astype(np.float32)[:, None]
    b_s = sB[G - 1, :].astype(np.float32)[None, :]
    ref = (S.astype(np.float32) * a_s * b_s).astype(np.float16)
    assert np.array_equal(f16bits(C), f16bits(ref))
    if N == 1:
        assert np.all(f16bits(C) == 0)


def _int4_groupwise_case(M, N, K, zfrac=False, pow2=False):
    G = (K + 127) // 128
    qA = RNG.integers(0, 16, (M, K))
    qB = RNG.integers(0, 16, (K, N))
    if pow2:
        sA = (2.0 ** -RNG.integers(0, 4, (M, G))).astype(np.float16)
        sB = (2.0 ** -RNG.integers(0, 4, (G, N))).astype(np.float16)
    else:
        sA = RNG.uniform(0.001, 0.02, (M, G)).astype(np.float16)
        sB = RNG.uniform(0.001, 0.02, (G, N)).astype(np.float16)
    zA = RNG.integers(0, 16, (M, G)).astype(np.float16)
    zB = RNG.integers(0, 16, (G, N)).astype(np.float16)
    if zfrac:
        zA = (zA + 0.5).astype(np.float16)  # ties round to even
        zB = (zB + 0.25).astype(np.float16)
    return qA, qB, sA, sB, zA, zB


@pytest.mark.parametrize("M,N,K,zfrac", [(6, 16, 256, False), (5, 3, 200, False), (4, 1, 384, True)])
def test_int4_groupwise_partials_and_value(M, N, K, zfrac):
    qA, qB, sA, sB, zA, zB = _int4_groupwise_case(M, N, K, zfrac)
    G = (K + 127) // 128
    A_q = pack_rows(qA)
    B_q = pack_cols(qB, (N + 1) // 2)
    C, out64, part = oracle.gemm_int4_groupwise(A_q, sA, zA, B_q, sB, zB, M, N, K,
                                                want_partials=True)
    zAi = np.rint(zA.astype(np.float64)).astype(np.int64)
    zBi = np.rint(zB.astype(np.float64)).astype(np.int64)
    ref_part = np.zeros((M, N, G), np.int64)
    ref = np.zeros((M, N), np.float64)
    for g in range(G):
        ks = slice(g * 128, min(K, (g + 1) * 128))
        va = qA[:, ks] - zAi[:, g:g + 1]
        vb = qB[ks, :] - zBi[g:g + 1, :]
        ref_part[:, :, g] = va @ vb
        ref += (sA[:, g].astype(np.float64)[:, None] * sB[g].astype(np.float64)[None, :]) * ref_part[:, :, g]
    assert np.array_equal(part.astype(np.int64), ref_part)
    assert np.allclose(out64, ref, rtol=1e-6, atol=1e-9)
    tol = 1e-2 * np.maximum(np.abs(ref), 1e-2 * np.sqrt(np.mean(ref ** 2)))
    assert np.all(np.abs(C.astype(np.float64) - ref) <= tol)


def test_int4_groupwise_pow2_scales_bit_exact():
    M, N, K = 8, 12, 512
    qA, qB, sA, sB, zA, zB = _int4_groupwise_case(M, N, K, pow2=True)
    C, out64, _ = oracle.gemm_int4_groupwise(pack_rows(qA), sA, zA, pack_cols(qB, N // 2),
                                             sB, zB, M, N, K)
    # power-of-two scales, small integers: every fp32 step is exact
    assert np.array_equal(f16bits(C), f16bits(out64.astype(np.float16)))


def test_int4_groupwise_equals_literal_when_zero8_and_constant_scales():
    M, N, K = 5, 8, 256
    G = 2
    qA = RNG.integers(0, 16, (M, K))
    qB = RNG.integers(0, 16, (K, N))
    sA = np.tile(RNG.uniform(0.001, 0.02, (M, 1)), (1, G)).astype(np.float16)
    sB = np.tile(RNG.uniform(0.001, 0.02, (1, N)), (G, 1)).astype(np.float16)
    z8a = np.full((M, G), 8, np.float16)
    z8b = np.full((G, N), 8, np.float16)
    Cg, _, _ = oracle.gemm_int4_groupwise(pack_rows(qA), sA, z8a, pack_cols(qB, N // 2), sB, z8b, M, N, K)
    Cl = oracle.gemm_int4_literal(pack_rows(qA), sA, pack_cols(qB, N // 2), sB, M, N, K)
    diff = np.abs(ordered(Cg) - ordered(Cl))
    assert diff.max() <= 1  # only fp32 association differs: at most one fp16 ulp


def test_w4a16_against_float64_dequant():
    T, O, K = 3, 20, 384
    G = K // 128
    X = RNG.standard_normal((T, K)).astype(np.float16)
    q = RNG.integers(0, 16, (O, K))
    s = RNG.uniform(0.001, 0.02, (O, G)).astype(np.float16)
    z = RNG.integers(0, 16, (O, G)).astype(np.float16)
    Yin = RNG.standard_normal((T, O)).astype(np.float16)
    W = (q - np.repeat(z.astype(np.float64), 128, axis=1)) * np.repeat(s.astype(np.float64), 128, axis=1)
    ref = X.astype(np.float64) @ W.T + Yin.astype(np.float64)
    Y, out64 = oracle.w4a16(X, pack_rows(q), s, z, Yin, alpha=1.0, beta=1.0)
    assert np.allclose(out64, ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(f16bits(Y), f16bits(out64.astype(np.float32).astype(np.float16)))


# ---- SwiGLU (src/kernels/activations.cu:9-11 silu_f, :76-134 swiglu_kernel) ----

def _swiglu_f64(g, u):
    """fp16(silu(g) * u) with silu and the product in float64, then one rounding
    to fp16 through fp32 (differs from the fp32 restatement only at rounding ties)"""
    g64 = g.astype(np.float64)
    s = g64 / (1.0 + np.exp(-g64))
    return (s * u.astype(np.float64)).astype(np.float32).astype(np.float16)


def test_swiglu_closed_forms():
    g = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 20.0, -20.0, 65504.0, -65504.0], np.float16)
    u = np.ones_like(g)
    out = oracle.swiglu(g, u).astype(np.float64)
    # silu(0) = 0, silu(x) -> x for x >> 0, silu(x) -> 0- for x << 0,
    # silu(1) = 1 / (1 + 1/e), silu(-1) = -1 / (1 + e)
    assert out[0] == 0.0 and out[1] == 0.0
    assert abs(out[2] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-3
    assert abs(out[3] + 1.0 / (1.0 + np.e)) < 1e-3
    assert abs(out[4] - 2.0 / (1.0 + np.exp(-2.0))) < 2e-3
    assert out[5] == 20.0 and out[7] == 65504.0
    assert -1e-7 < out[6] < 0.0 and out[8] == 0.0  # exp(65504) overflows: -65504 / inf = -0
    # linear in up
    g2 = RNG.standard_normal(64).astype(np.float16)
    one = oracle.swiglu(g2, np.ones_like(g2))
    assert np.array_equal(f16bits(oracle.swiglu(g2, np.full_like(g2, 2.0))),
                          f16bits((one.astype(np.float32) * 2).astype(np.float16)))


def test_swiglu_against_float64_formula():
    n = 1 << 16
    g = (RNG.standard_normal(n) * 4).astype(np.float16)
    u = (RNG.standard_normal(n) * 2).astype(np.float16)
    out = oracle.swiglu(g, u)
    ref = _swiglu_f64(g, u)
    d = np.abs(f16bits(out).astype(np.int32) - f16bits(ref).astype(np.int32))
    # fp32 intermediates: at most one fp16 ulp, and only at rounding boundaries
    assert d.max() <= 1 and np.count_nonzero(d) < n // 1000
    # a restatement with the sign of the exponent flipped is caught
    bad = (g.astype(np.float64) / (1.0 + np.exp(g.astype(np.float64))) * u).astype(np.float16)
    assert np.count_nonzero(f16bits(bad) != f16bits(out)) > n // 2


def test_w4a16_swiglu_is_gate_up_then_swiglu():
    T, I, K = 3, 24, 256
    G = K // 128
    X = RNG.standard_normal((T, K)).astype(np.float16)
    q = RNG.integers(0, 16, (2 * I, K))
    s = RNG.uniform(0.001, 0.02, (2 * I, G)).astype(np.float16)
    z = RNG.integers(0, 16, (2 * I, G)).astype(np.float16)
    H = oracle.w4a16_swiglu(X, pack_rows(q), s, z)
    W = (q - np.repeat(z.astype(np.float64), 128, axis=1)) * np.repeat(s.astype(np.float64), 128, axis=1)
    lin = X.astype(np.float64) @ W.T
    gate = lin[:, :I].astype(np.float32).astype(np.float16)
    up = lin[:, I:].astype(np.float32).astype(np.float16)
    assert H.shape == (T, I)
    d = np.abs(f16bits(H).astype(np.int32) - f16bits(_swiglu_f64(gate, up)).astype(np.int32))
    assert d.max() <= 1
