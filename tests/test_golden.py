"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle).

CPU: the oracle still reproduces every fixture bit for bit, and each fixture
agrees with numpy where the arithmetic pins it (integer accumulators exactly,
the float64 values to rounding, the fp16 outputs within the stated tolerance
of float64).  GPU: the HIP library reproduces the fixtures through the C ABI,
bit-exact for INT8 and INT4-literal, within tolerance for the rest.
"""
import glob
import os

import numpy as np
import pytest

import oracle
from tests._util import f16bits, to_dev, to_host, within_tol

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
        return {k: z[k] for k in z.files}


def nibbles_rows(p, K):
    """[R, K/2] bytes -> [R, K] values, high nibble = even k (gemm_int4.cu:27-34)."""
    p = np.asarray(p, np.uint8)
    q = np.empty((p.shape[0], 2 * p.shape[1]), np.int64)
    q[:, 0::2] = p >> 4
    q[:, 1::2] = p & 15
    return q[:, :K]


def nibbles_cols(p, N):
    """[K, ceil(N/2)] bytes -> [K, N] values, high nibble = even n."""
    p = np.asarray(p, np.uint8)
    q = np.empty((p.shape[0], 2 * p.shape[1]), np.int64)
    q[:, 0::2] = p >> 4
    q[:, 1::2] = p & 15
    return q[:, :N]


def _groups(K):
    return (K + 127) // 128


def test_fixtures_present():
    assert len(NAMES) >= 11, NAMES


# ---------------------------------------------------------------------------
# CPU: the oracle reproduces the fixtures
# ---------------------------------------------------------------------------
def oracle_outputs(name, f):
    if name.startswith("fp16_batched"):
        return {"C": oracle.gemm_fp16_batched(f["A"], f["B"], None, float(f["alpha"]), float(f["beta"])),
                "C64": np.stack([oracle.gemm_fp16_f64(a, b) for a, b in zip(f["A"], f["B"])])}
    if name.startswith("fp16"):
        a, b = float(f["alpha"]), float(f["beta"])
        return {"C": oracle.gemm_fp16(f["A"], f["B"], f["C_in"], a, b),
                "C64": oracle.gemm_fp16_f64(f["A"], f["B"], f["C_in"], a, b)}
    if name.startswith("int8_tensor"):
        C, acc = oracle.gemm_int8(f["A"], f["B"], float(f["A_scale"]), int(f["A_zero"]),
                                  float(f["B_scale"]), int(f["B_zero"]))
        return {"C": C, "acc": acc}
    if name.startswith("int8_rowcol"):
        C, acc = oracle.gemm_int8_rowcol(f["A"], f["B"], f["sa"], f["sb"])
        return {"C": C, "acc": acc}
    if name.startswith("int4_literal"):
        M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
        return {"C": oracle.gemm_int4_literal(f["A_q"], f["A_scale"], f["B_q"], f["B_scale"], M, N, K)}
    if name.startswith("int4_groupwise"):
        M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
        C, C64, part = oracle.gemm_int4_groupwise(f["A_q"], f["A_scale"], f["A_zero"], f["B_q"],
                                                  f["B_scale"], f["B_zero"], M, N, K, want_partials=True)
        return {"C": C, "C64": C64, "partials": part}
    if name.startswith("w4a16_swiglu"):
        return {"H": oracle.w4a16_swiglu(f["X"], f["W_q"], f["W_scale"], f["W_zero"])}
    if name.startswith("w4a16"):
        Y, Y64 = oracle.w4a16(f["X"], f["W_q"], f["W_scale"], f["W_zero"], f["Y_in"],
                              float(f["alpha"]), float(f["beta"]))
        return {"Y": Y, "Y64": Y64}
    if name.startswith("swiglu"):
        return {"out": oracle.swiglu(f["gate"], f["up"])}
    raise KeyError(name)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    f = load(name)
    for key, got in oracle_outputs(name, f).items():
        want = f[key]
        assert got.dtype == want.dtype and got.shape == want.shape, key
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"{name}: {key} differs"


# ---------------------------------------------------------------------------
# CPU: the fixtures against numpy
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name", [n for n in NAMES if n.startswith("fp16") and "batched" not in n])
def test_fp16_fixture_against_numpy(name):
    f = load(name)
    a, b = float(f["alpha"]), float(f["beta"])
    ref = a * (f["A"].astype(np.float64) @ f["B"].astype(np.float64)) + b * f["C_in"].astype(np.float64)
    np.testing.assert_allclose(f["C64"], ref, rtol=1e-12, atol=1e-12)
    ok, rep = within_tol(f["C"], ref)
    assert ok, rep


def test_fp16_batched_fixture_against_numpy():
    f = load("fp16_batched_3x5x24x40")
    ref = np.matmul(f["A"].astype(np.float64), f["B"].astype(np.float64))
    np.testing.assert_allclose(f["C64"], ref, rtol=1e-12, atol=1e-12)
    ok, rep = within_tol(f["C"], ref)
    assert ok, rep


def _int8_epilogue(acc, s):
    return (acc.astype(np.float32) * np.float32(s)).astype(np.float16)


def test_int8_tensor_fixture_against_numpy():
    f = load("int8_tensor_17x40x64")
    A = f["A"].astype(np.int64) - int(f["A_zero"])
    B = f["B"].astype(np.int64) - int(f["B_zero"])
    acc = (A @ B).astype(np.int32)
    assert np.array_equal(f["acc"], acc)
    s = np.float32(f["A_scale"]) * np.float32(f["B_scale"])
    assert np.array_equal(f16bits(f["C"]), f16bits(_int8_epilogue(acc, s)))


def test_int8_rowcol_fixture_against_numpy():
    f = load("int8_rowcol_16x24x96")
    acc = (f["A"].astype(np.int64) @ f["B"].astype(np.int64)).astype(np.int32)
    assert np.array_equal(f["acc"], acc)
    s = f["sa"].astype(np.float32)[:, None] * f["sb"].astype(np.float32)[None, :]
    C = (acc.astype(np.float32) * s).astype(np.float16)
    assert np.array_equal(f16bits(f["C"]), f16bits(C))


def test_int4_literal_fixture_against_numpy():
    # the reference's arithmetic (gemm_int4.cu:81-190): q - 8, zeros ignored, the
    # whole-K integer sum scaled by the LAST group's scales of A and B
    f = load("int4_literal_16x5x256")
    M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
    G = _groups(K)
    qa = nibbles_rows(f["A_q"], K) - 8
    assert f["B_q"].shape == (K, N // 2)  # the reference's [K, N/2] layout
    qb = np.zeros((K, N), np.int64)       # odd N: the last column is never loaded
    qb[:, :2 * (N // 2)] = nibbles_cols(f["B_q"], 2 * (N // 2)) - 8
    S = (qa @ qb).astype(np.float32)
    C = ((S * f["A_scale"][:, G - 1].astype(np.float32)[:, None])
         * f["B_scale"][G - 1, :].astype(np.float32)[None, :]).astype(np.float16)
    assert np.array_equal(f16bits(f["C"]), f16bits(C))


def test_int4_groupwise_fixture_against_numpy():
    f = load("int4_groupwise_16x3x384")
    M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
    G = _groups(K)
    qa = nibbles_rows(f["A_q"], K)
    qb = nibbles_cols(f["B_q"], N)
    ref = np.zeros((M, N))
    for g in range(G):
        ks = slice(128 * g, min(K, 128 * g + 128))
        da = qa[:, ks] - np.rint(f["A_zero"][:, g].astype(np.float64)).astype(np.int64)[:, None]
        db = qb[ks, :] - np.rint(f["B_zero"][g, :].astype(np.float64)).astype(np.int64)[None, :]
        P = da @ db
        assert np.array_equal(f["partials"][:, :, g], P.astype(np.int32))
        ref += P * f["A_scale"][:, g].astype(np.float64)[:, None] * f["B_scale"][g, :].astype(np.float64)[None, :]
    np.testing.assert_allclose(f["C64"], ref, rtol=1e-12, atol=1e-15)
    ok, rep = within_tol(f["C"], ref)
    assert ok, rep


def _dequant(W_q, s, z, K):
    q = nibbles_rows(W_q, K).astype(np.float64)
    G = _groups(K)
    idx = np.arange(K) // 128
    assert idx.max() < G
    return (q - z.astype(np.float64)[:, idx]) * s.astype(np.float64)[:, idx]


def test_w4a16_fixture_against_numpy():
    f = load("w4a16_3x40x256_residual")
    K = f["X"].shape[1]
    W = _dequant(f["W_q"], f["W_scale"], f["W_zero"], K)
    ref = float(f["alpha"]) * (f["X"].astype(np.float64) @ W.T) + float(f["beta"]) * f["Y_in"].astype(np.float64)
    np.testing.assert_allclose(f["Y64"], ref, rtol=1e-12, atol=1e-12)
    ok, rep = within_tol(f["Y"], ref)
    assert ok, rep


def _silu_mul64(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


def _ulps(a, b):
    a = a.astype(np.float16).view(np.int16).astype(np.int64)
    b = b.astype(np.float16).view(np.int16).astype(np.int64)
    a = np.where(a < 0, -32768 - a, a)
    b = np.where(b < 0, -32768 - b, b)
    return np.abs(a - b)


def test_swiglu_fixture_against_numpy():
    f = load("swiglu_1000")
    ref = _silu_mul64(f["gate"], f["up"]).astype(np.float16)
    assert _ulps(f["out"], ref).max() <= 1


def test_w4a16_swiglu_fixture_against_numpy():
    f = load("w4a16_swiglu_2x24x256")
    I, K = int(f["I"]), f["X"].shape[1]
    W = _dequant(f["W_q"], f["W_scale"], f["W_zero"], K)
    X = f["X"].astype(np.float64)
    gate = (X @ W[:I].T).astype(np.float16)
    up = (X @ W[I:].T).astype(np.float16)
    ref = _silu_mul64(gate, up)
    ok, rep = within_tol(f["H"], ref)
    assert ok, rep


# ---------------------------------------------------------------------------
# GPU: the HIP library against the fixtures, through the C ABI
# ---------------------------------------------------------------------------
def _cg():
    import clove_compute_amd as cg
    return cg


def _run(name, f):
    import torch
    cg = _cg()
    if name.startswith("fp16_batched"):
        bt, M, K = f["A"].shape
        N = f["B"].shape[2]
        C = torch.zeros(bt, M, N, dtype=torch.float16, device="cuda")
        cg.gemm_fp16_batched(to_dev(f["A"]), to_dev(f["B"]), C, bt, M, N, K, float(f["alpha"]), float(f["beta"]))
        return {"C": C}
    if name.startswith("fp16"):
        M, K = f["A"].shape
        N = f["B"].shape[1]
        C = to_dev(f["C_in"])
        cg.gemm_fp16(to_dev(f["A"]), to_dev(f["B"]), C, M, N, K, float(f["alpha"]), float(f["beta"]))
        return {"C": C}
    if name.startswith("int8_tensor"):
        M, K = f["A"].shape
        N = f["B"].shape[1]
        C = torch.empty(M, N, dtype=torch.float16, device="cuda")
        acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
        A, B = to_dev(f["A"]), to_dev(f["B"])
        cg.gemm_int8(A, B, C, M, N, K, float(f["A_scale"]), int(f["A_zero"]), float(f["B_scale"]), int(f["B_zero"]))
        cg.gemm_int8_acc32(A, B, acc, M, N, K, int(f["A_zero"]), int(f["B_zero"]))
        return {"C": C, "acc": acc}
    if name.startswith("int8_rowcol"):
        M, K = f["A"].shape
        N = f["B"].shape[1]
        C = torch.empty(M, N, dtype=torch.float16, device="cuda")
        acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
        A, B = to_dev(f["A"]), to_dev(f["B"])
        cg.gemm_int8_rowcol(A, B, to_dev(f["sa"]), to_dev(f["sb"]), C, M, N, K)
        cg.gemm_int8_acc32(A, B, acc, M, N, K)
        return {"C": C, "acc": acc}
    if name.startswith("int4"):
        M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
        C = torch.empty(M, N, dtype=torch.float16, device="cuda")
        mode = cg.CLOVE_INT4_REFERENCE_LITERAL if "literal" in name else cg.CLOVE_INT4_GROUPWISE
        cg.gemm_int4_ex(to_dev(f["A_q"]), to_dev(f["A_scale"]), to_dev(f["A_zero"]), to_dev(f["B_q"]),
                        to_dev(f["B_scale"]), to_dev(f["B_zero"]), C, M, N, K, mode)
        return {"C": C}
    if name.startswith("w4a16_swiglu"):
        T, K = f["X"].shape
        I = int(f["I"])
        H = torch.empty(T, I, dtype=torch.float16, device="cuda")
        cg.w4a16_swiglu(to_dev(f["X"]), to_dev(f["W_q"]), to_dev(f["W_scale"]), to_dev(f["W_zero"]), H, T, I, K)
        return {"H": H}
    if name.startswith("w4a16"):
        T, K = f["X"].shape
        O = f["W_q"].shape[0]
        Y = to_dev(f["Y_in"])
        cg.gemm_w4a16(to_dev(f["X"]), to_dev(f["W_q"]), to_dev(f["W_scale"]), to_dev(f["W_zero"]), Y, T, O, K,
                      float(f["alpha"]), float(f["beta"]))
        return {"Y": Y}
    if name.startswith("swiglu"):
        out = torch.empty(f["gate"].shape[0], dtype=torch.float16, device="cuda")
        cg.swiglu(to_dev(f["gate"]), to_dev(f["up"]), out, f["gate"].shape[0])
        return {"out": out}
    raise KeyError(name)


# fp16 outputs compared within tolerance of this float64 key (None: of the oracle's fp16 output)
_TOL_REF = {"fp16": "C64", "int4_groupwise": "C64", "w4a16_3": "Y64"}


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_library_matches_fixture(name):
    import torch
    print(f"golden case {name}", flush=True)
    f = load(name)
    got = {k: to_host(v) for k, v in _run(name, f).items()}
    torch.cuda.synchronize()
    for key, g in got.items():
        want = f[key]
        assert g.shape == want.shape, (key, g.shape, want.shape)
        if name.startswith("int8") or name.startswith("int4_literal"):
            assert np.array_equal(g.view(np.uint8), want.view(np.uint8)), f"{name}: {key} not bit-exact"
        elif name.startswith("swiglu"):
            assert _ulps(g, want).max() <= 1, name
        else:
            ref_key = next((v for k, v in _TOL_REF.items() if name.startswith(k)), None)
            ref = f[ref_key] if ref_key is not None else want.astype(np.float64)
            ok, rep = within_tol(g, ref)
            assert ok, (name, key, rep)
