"""GPU parity of clove_gemm_w4a16 (fp16 activations x group-128 INT4 weights).

Shapes: the Llama-style 1B decoder layer (hidden 2048, 32 q / 8 kv heads of 64:
QKV 2048->3072, O 2048->2048, gate/up 2048->8192, down 8192->2048) at token
batch 1 and 512, O and down with the beta = 1 residual the reference runtime
uses (src/runtime/inference.cu:165-168, :191-194).
"""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, f16bits, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu

LAYER = [("qkv", 3072, 2048, 0.0), ("o", 2048, 2048, 1.0), ("gate", 8192, 2048, 0.0),
         ("up", 8192, 2048, 0.0), ("down", 2048, 8192, 1.0)]


def _cg():
    import clove_compute_amd as cg
    return cg


def make(T, O, K, key, pow2=False):
    g = rng("w4a16", T, O, K, key)
    G = (K + 127) // 128
    if pow2:
        X = g.integers(-3, 4, (T, K)).astype(np.float16)
        q = g.integers(6, 11, (O, K))
        s = (2.0 ** -g.integers(0, 3, (O, G))).astype(np.float16)
        z = np.full((O, G), 8, np.float16)
    else:
        X = g.standard_normal((T, K)).astype(np.float16)
        q = g.integers(0, 16, (O, K))
        s = g.uniform(0.001, 0.02, (O, G)).astype(np.float16)
        z = g.integers(0, 16, (O, G)).astype(np.float16)
    from clove_compute_amd import quant
    return X, quant.pack_rows(q), s, z, g


def run(X, W, s, z, Yin, O, alpha=1.0, beta=0.0):
    import torch
    T, K = X.shape
    Y = to_dev(Yin) if Yin is not None else empty_f16(T, O, fill=float("nan"))
    _cg().gemm_w4a16(to_dev(X), to_dev(W), to_dev(s), to_dev(z), Y, T, O, K, alpha, beta)
    torch.cuda.synchronize()
    return to_host(Y)


@pytest.mark.parametrize("T", [1, 512])
@pytest.mark.parametrize("name,O,K,beta", LAYER)
def test_llama1b_layer(T, name, O, K, beta):
    X, W, s, z, g = make(T, O, K, name)
    Yin = g.standard_normal((T, O)).astype(np.float16) if beta else None
    Y = run(X, W, s, z, Yin, O, 1.0, beta)
    rows = np.arange(T) if T <= 4 else np.unique(np.concatenate([[0, T - 1], g.integers(0, T, 12)]))
    _, ref = oracle.w4a16(X[rows], W, s, z, None if Yin is None else Yin[rows], 1.0, beta)
    ok, rep = within_tol(Y[rows], ref)
    assert ok, (name, rep)


@pytest.mark.parametrize("T,O,K", [(1, 1024, 2048), (1, 3000, 4096), (1, 2048, 11008), (2, 2048, 8192),
                                   (4, 2048, 4096), (3, 520, 1024),
                                   (4, 256, 8192), (64, 512, 1024),
                                   (300, 136, 256), (4, 300, 11008), (2, 520, 16384),
                                   (1, 6000, 2048), (1, 1031, 4096), (1, 2051, 8192), (1, 1000, 16384),
                                   (1, 130, 2080), (1, 70, 16416)])
def test_pow2_bit_exact(T, O, K):
    # (T = 2..4 on long rows: more X pieces than the GEMV's prefetch holds;
    # one token: X per lane in registers with one to four rows per wave (6000
    # rows: two), and the waves of a workgroup splitting K with one, two or
    # four rows per workgroup, the last one ragged (1031, 2051), up to eight
    # waves (K = 16384); the bounds of that form: 65 chunks, the second wave
    # holding one (K = 2080), and 513 chunks, past it (K = 16416))
    X, W, s, z, _ = make(T, O, K, "pow2", pow2=True)
    Y = run(X, W, s, z, None, O)
    _, ref = oracle.w4a16(X, W, s, z)
    assert np.array_equal(f16bits(Y), f16bits(ref.astype(np.float16)))


@pytest.mark.parametrize("T,O,K", [(1, 77, 200), (2, 33, 96), (5, 45, 330), (70, 70, 64), (1, 8, 11008)])
def test_ragged(T, O, K):
    X, W, s, z, g = make(T, O, K, "ragged")
    Yin = g.standard_normal((T, O)).astype(np.float16)
    Y = run(X, W, s, z, Yin, O, 0.5, 1.0)
    _, ref = oracle.w4a16(X, W, s, z, Yin, 0.5, 1.0)
    ok, rep = within_tol(Y, ref)
    assert ok, rep


# K % 128 == 0 and T > 4 take the INT4-weight MFMA kernel (i4w_gemm): every
# tile configuration (X rows <= 32, <= 64, 128 x 128, 256 x 128), ragged
# token and weight-row counts, split K, alpha/beta
@pytest.mark.parametrize("T,O,K", [(6, 1000, 4096), (37, 300, 1024), (100, 200, 2048), (257, 129, 384),
                                   (1024, 8192, 256), (512, 3072, 2048)])
def test_mfma_path_shapes(T, O, K):
    X, W, s, z, g = make(T, O, K, "mfma")
    Yin = g.standard_normal((T, O)).astype(np.float16)
    Y = run(X, W, s, z, Yin, O, 0.5, 1.0)
    rows = np.arange(T) if T <= 300 else np.unique(np.concatenate([[0, T - 1], g.integers(0, T, 24)]))
    _, ref = oracle.w4a16(X[rows], W, s, z, Yin[rows], 0.5, 1.0)
    ok, rep = within_tol(Y[rows], ref)
    assert ok, rep


@pytest.mark.parametrize("T,O,K", [(6, 1000, 4096), (200, 640, 1024), (1024, 8192, 256)])
def test_mfma_path_pow2_bit_exact(T, O, K):
    X, W, s, z, _ = make(T, O, K, "pow2m", pow2=True)
    Y = run(X, W, s, z, None, O)
    _, ref = oracle.w4a16(X, W, s, z)
    assert np.array_equal(f16bits(Y), f16bits(ref.astype(np.float16)))


# 5..32 tokens with K % 128 == 0 take the streaming kernel (i4w_stream.hpp):
# every K-slice configuration (G = 1, 10, 20, 30, 40, 60, 86 groups: 2, 4 or 8
# waves of up to 8 or 11 groups, waves without groups when G is small), one
# and two 16-token fragments, one and two 16-row weight fragments per
# workgroup (8192 rows), ragged weight rows, alpha/beta
@pytest.mark.parametrize("T,O,K", [(5, 77, 128), (16, 300, 1280), (17, 130, 2560), (32, 1000, 3840),
                                   (8, 8192, 5120), (31, 8192, 7680), (12, 4096, 11008 // 128 * 128),
                                   (3, 4096, 4096), (4, 1024, 11008 // 128 * 128)])
def test_stream_path_shapes(T, O, K):
    # (T = 3, 4 on weights above 8 Mi elements take the streaming kernel too)
    X, W, s, z, g = make(T, O, K, "stream")
    Yin = g.standard_normal((T, O)).astype(np.float16)
    Y = run(X, W, s, z, Yin, O, 0.75, 0.5)
    _, ref = oracle.w4a16(X, W, s, z, Yin, 0.75, 0.5)
    ok, rep = within_tol(Y, ref)
    assert ok, rep


@pytest.mark.parametrize("T,O,K", [(6, 200, 1024), (32, 96, 11008 // 128 * 128)])
def test_stream_path_pow2_bit_exact(T, O, K):
    X, W, s, z, _ = make(T, O, K, "pow2s", pow2=True)
    Y = run(X, W, s, z, None, O)
    _, ref = oracle.w4a16(X, W, s, z)
    assert np.array_equal(f16bits(Y), f16bits(ref.astype(np.float16)))
