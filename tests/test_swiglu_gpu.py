"""GPU parity of the SwiGLU entry points.

* clove_swiglu -- the reference's elementwise swiglu (src/kernels/activations.cu:76-134)
* clove_w4a16_swiglu -- the MLP's gate and up projections and SwiGLU
  (src/runtime/inference.cu:172-186) on one fused INT4 weight [2I, K/2]: the
  GEMV for T <= 4, the INT4-weight MFMA GEMM (gate and up rows of one output
  met inside a workgroup) for larger T, the two W4A16 layers and the
  elementwise pass for K % 128 != 0 or unaligned operands
* clove_swiglu_fused -- the reference's declared swiglu_fused
  (include/clove/kernels/activations.cuh:37-46) on FP16 weights, one launch
  with no intermediate buffer, bit-identical to two gemm_fp16 calls and
  swiglu on the shapes where those take the same kernel family

The checker is the oracle: swiglu restated in C (fp32 silu with libm expf),
W4A16 in float64.  Device expf and libm expf may differ by an fp32 ulp, which
can move an fp16 result by one ulp at a rounding boundary: the elementwise
comparison allows that, and nothing more.
"""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, f16bits, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu


def _cg():
    import clove_compute_amd as cg
    return cg


def _sync():
    import torch
    torch.cuda.synchronize()


def ulp_diff(a, b):
    """|a - b| in fp16 ulps for finite values of equal sign (sign-magnitude bits)"""
    ia = f16bits(a).astype(np.int32)
    ib = f16bits(b).astype(np.int32)
    ia = np.where(ia & 0x8000, -(ia & 0x7fff), ia)
    ib = np.where(ib & 0x8000, -(ib & 0x7fff), ib)
    return np.abs(ia - ib)


def assert_swiglu_close(got, ref):
    d = ulp_diff(got, ref)
    assert d.max() <= 1, int(d.max())
    assert np.count_nonzero(d) <= max(2, d.size // 1000), int(np.count_nonzero(d))


# ---- elementwise ----

@pytest.mark.parametrize("n", [1, 7, 8, 1000, 4097, 1 << 20])
@pytest.mark.parametrize("inplace", [False, True])
def test_swiglu_elementwise(n, inplace):
    import torch
    g = rng("swiglu", n)
    gate = (g.standard_normal(n) * 4).astype(np.float16)
    up = (g.standard_normal(n) * 2).astype(np.float16)
    dg, du = to_dev(gate), to_dev(up)
    out = dg if inplace else empty_f16(n, fill=float("nan"))
    _cg().swiglu(dg, du, out, n)
    _sync()
    assert_swiglu_close(to_host(out), oracle.swiglu(gate, up))


def test_swiglu_elementwise_unaligned_and_special_values():
    import torch
    vals = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 65504.0, -65504.0, 11.0, -11.0, 0.5], np.float16)
    gate = np.concatenate([vals, np.random.default_rng(5).standard_normal(1000).astype(np.float16)])
    up = np.full_like(gate, 1.5)
    n = gate.size
    # views one element into larger buffers: 2-byte aligned, not 16
    bg = to_dev(np.concatenate([np.zeros(1, np.float16), gate]))
    bu = to_dev(np.concatenate([np.zeros(1, np.float16), up]))
    bo = empty_f16(n + 1, fill=float("nan"))
    cg = _cg()
    cg.swiglu(bg.data_ptr() + 2, bu.data_ptr() + 2, bo.data_ptr() + 2, n)
    _sync()
    got = to_host(bo)[1:]
    assert_swiglu_close(got, oracle.swiglu(gate, up))
    assert got[0] == 0.0 and got[4] == np.float16(30.0)


# ---- fused INT4 gate/up + SwiGLU ----

def make_gate_up(T, I, K, key, pow2=False):
    g = rng("w4a16_swiglu", T, I, K, key)
    G = (K + 127) // 128
    if pow2:
        # small integers and power-of-two scales: gate and up exact in fp32
        X = g.integers(-3, 4, (T, K)).astype(np.float16)
        q = g.integers(6, 11, (2 * I, K))
        s = (2.0 ** -g.integers(2, 5, (2 * I, G))).astype(np.float16)
        z = np.full((2 * I, G), 8, np.float16)
    else:
        X = g.standard_normal((T, K)).astype(np.float16)
        q = g.integers(0, 16, (2 * I, K))
        s = g.uniform(0.001, 0.02, (2 * I, G)).astype(np.float16)
        z = g.integers(0, 16, (2 * I, G)).astype(np.float16)
    from clove_compute_amd import quant
    return X, quant.pack_rows(q), s, z, g


def run_w4a16_swiglu(X, Wq, s, z, I, x_offset=False):
    import torch
    T, K = X.shape
    if x_offset:
        buf = to_dev(np.concatenate([np.zeros(1, np.float16), X.reshape(-1)]))
        xp = buf.data_ptr() + 2
    else:
        dX = to_dev(X)
        xp = dX
    H = empty_f16(T, I, fill=float("nan"))
    dW, ds, dz = to_dev(Wq), to_dev(s), to_dev(z)
    _cg().w4a16_swiglu(xp, dW, ds, dz, H, T, I, K)
    _sync()
    return to_host(H)


def check_rows(X, Wq, s, z, H, rows):
    ref = oracle.w4a16_swiglu(X[rows], Wq, s, z)
    ok, rep = within_tol(H[rows], ref.astype(np.float64))
    assert ok, rep


# T <= 4: GEMV; T > 4 with K % 128 == 0: the MFMA GEMM (64x32 tiles up to 32
# tokens, 128x64 / 256x128 above, with and without split K; from 512 tokens
# 256x64, or 256x128 with eight waves where those tiles cover 3/4 of the CUs:
# the Llama-1B MLP at T = 512 and the ragged 1000 x 3000); the Llama-1B MLP
# (I = 8192, K = 2048) at decode and prefill
@pytest.mark.parametrize("T,I,K", [(1, 8192, 2048), (2, 300, 1024), (3, 64, 256), (4, 1000, 4096),
                                   (5, 8192, 2048), (17, 200, 512), (33, 1000, 1024), (64, 96, 2048),
                                   (100, 777, 384), (512, 8192, 2048), (1, 2000, 4096), (1, 1100, 8192),
                                   (600, 520, 1024), (1030, 136, 256), (1000, 3000, 256)])
def test_w4a16_swiglu_shapes(T, I, K):
    X, Wq, s, z, g = make_gate_up(T, I, K, "shapes")
    H = run_w4a16_swiglu(X, Wq, s, z, I)
    rows = np.unique(np.concatenate([[0, T - 1], g.integers(0, T, min(T, 8))]))
    check_rows(X, Wq, s, z, H, rows)
    assert np.all(np.isfinite(H.astype(np.float32)))


# shapes outside the fused kernels' domain: two W4A16 layers + SwiGLU
@pytest.mark.parametrize("T,I,K,x_offset", [(40, 128, 200, False), (9, 64, 256, True)])
def test_w4a16_swiglu_composed_fallback(T, I, K, x_offset):
    X, Wq, s, z, g = make_gate_up(T, I, K, "fallback")
    H = run_w4a16_swiglu(X, Wq, s, z, I, x_offset=x_offset)
    check_rows(X, Wq, s, z, H, np.arange(T))


@pytest.mark.parametrize("T,I,K", [(1, 512, 1024), (4, 96, 256), (48, 256, 512), (300, 640, 768),
                                   (512, 640, 768), (1024, 3072, 256)])
def test_w4a16_swiglu_exact_inputs(T, I, K):
    # gate and up are exact: the only freedom left is expf's last fp32 bit
    X, Wq, s, z, _ = make_gate_up(T, I, K, "pow2", pow2=True)
    H = run_w4a16_swiglu(X, Wq, s, z, I)
    assert_swiglu_close(H, oracle.w4a16_swiglu(X, Wq, s, z))


def test_w4a16_swiglu_k_zero():
    cg = _cg()
    H = empty_f16(3, 5, fill=float("nan"))
    dummy = to_dev(np.zeros(16, np.float16))
    cg.w4a16_swiglu(dummy, dummy, dummy, dummy, H, 3, 5, 0)
    _sync()
    assert np.all(to_host(H) == 0)


def test_w4a16_swiglu_equals_layers_then_swiglu():
    # the same numbers through the unfused route: gate and up layers, then swiglu
    import torch
    T, I, K = 24, 384, 1024
    X, Wq, s, z, _ = make_gate_up(T, I, K, "compose", pow2=True)
    cg = _cg()
    dX = to_dev(X)
    gate = empty_f16(T, I)
    up = empty_f16(T, I)
    cg.gemm_w4a16(dX, to_dev(Wq[:I]), to_dev(s[:I]), to_dev(z[:I]), gate, T, I, K)
    cg.gemm_w4a16(dX, to_dev(Wq[I:]), to_dev(s[I:]), to_dev(z[I:]), up, T, I, K)
    H2 = empty_f16(T, I)
    cg.swiglu(gate, up, H2, T * I)
    _sync()
    H = run_w4a16_swiglu(X, Wq, s, z, I)
    assert np.array_equal(f16bits(H), f16bits(to_host(H2)))


# ---- FP16 swiglu_fused (the reference's declaration) ----
# One launch, no intermediate: the FP16 GEMV with two weight operands for
# T <= 4, the skinny MFMA kernel with two B operands for T > 4 (every tile
# shape: 32x128, 128x64, 64x64, 128x128 with and without K splits),
# and the direct fallback for unaligned operands or hidden % 64 != 0.

def run_swiglu_fused(X, Wg, Wu, offset=False):
    T, H = X.shape
    I = Wg.shape[1]
    if offset:
        # 2-byte aligned views one element into larger buffers
        bx = to_dev(np.concatenate([np.zeros(1, np.float16), X.reshape(-1)]))
        bg = to_dev(np.concatenate([np.zeros(1, np.float16), Wg.reshape(-1)]))
        bu = to_dev(np.concatenate([np.zeros(1, np.float16), Wu.reshape(-1)]))
        bo = empty_f16(T * I + 1, fill=float("nan"))
        _cg().swiglu_fused(bx.data_ptr() + 2, bg.data_ptr() + 2, bu.data_ptr() + 2, bo.data_ptr() + 2, T, H, I)
        _sync()
        return to_host(bo)[1:].reshape(T, I)
    out = empty_f16(T, I, fill=float("nan"))
    _cg().swiglu_fused(to_dev(X), to_dev(Wg), to_dev(Wu), out, T, H, I)
    _sync()
    return to_host(out)


def make_mlp(T, H, I, key):
    g = rng("swiglu_fused", key, T, H, I)
    X = g.standard_normal((T, H)).astype(np.float16)
    Wg = (g.standard_normal((H, I)) * 0.05).astype(np.float16)
    Wu = (g.standard_normal((H, I)) * 0.05).astype(np.float16)
    return X, Wg, Wu, g


@pytest.mark.parametrize("T,H,I", [(1, 2048, 8192), (3, 512, 1000), (7, 64, 96), (40, 1024, 520),
                                   (64, 512, 1000), (128, 512, 1000), (300, 512, 768),
                                   (512, 2048, 8192), (1024, 512, 4096)])
def test_swiglu_fused_fp16(T, H, I):
    X, Wg, Wu, g = make_mlp(T, H, I, "tol")
    got = run_swiglu_fused(X, Wg, Wu)
    rows = np.unique(np.concatenate([[0, T - 1], g.integers(0, T, min(T, 8))]))
    gate = oracle.gemm_fp16_f64(X[rows], Wg).astype(np.float32).astype(np.float16)
    up = oracle.gemm_fp16_f64(X[rows], Wu).astype(np.float32).astype(np.float16)
    ok, rep = within_tol(got[rows], oracle.swiglu(gate, up).astype(np.float64))
    assert ok, rep


@pytest.mark.parametrize("T,H,I", [(1, 2048, 8192), (2, 1024, 512), (4, 4096, 264), (7, 64, 96),
                                   (40, 1024, 520), (64, 512, 1000), (128, 4096, 1024), (300, 512, 768),
                                   (512, 2048, 8192), (3, 4096, 4096), (2, 4096, 11008),
                                   (1024, 2048, 8192), (2048, 4096, 11008), (96, 4096, 10240)])
def test_swiglu_fused_equals_gemms_then_swiglu(T, H, I):
    # the fused kernels sum gate and up in the order gemm_fp16 does for the
    # same shape (same kernel family, tiles and split plan: the GEMV, or the
    # skinny kernel for T > 4 and for T = 2..4 on large weights), so the result
    # is the two GEMMs followed by swiglu, bit for bit; where gemm_fp16 takes
    # its 256x256 tile (1024 x 2048 x 8192 and 2048 x 4096 x 11008: the tiles of
    # [T, I] cover half the CUs) the fused call is those two GEMMs and swiglu
    X, Wg, Wu, _ = make_mlp(T, H, I, "bits")
    got = run_swiglu_fused(X, Wg, Wu)
    cg = _cg()
    dX = to_dev(X)
    gate, up, ref = empty_f16(T, I), empty_f16(T, I), empty_f16(T, I)
    cg.gemm_fp16(dX, to_dev(Wg), gate, T, I, H)
    cg.gemm_fp16(dX, to_dev(Wu), up, T, I, H)
    cg.swiglu(gate, up, ref, T * I)
    _sync()
    assert np.array_equal(f16bits(got), f16bits(to_host(ref)))


@pytest.mark.parametrize("T,H,I,offset", [(5, 60, 100, False), (3, 100, 30, False), (33, 200, 72, False),
                                          (2, 256, 128, True), (20, 128, 64, True)])
def test_swiglu_fused_direct_fallback(T, H, I, offset):
    # outside the fast kernels' domain: fp32 fmaf over k in order for both
    # projections, which is the oracle's naive-kernel arithmetic bit for bit;
    # only expf's last fp32 bit is left free
    X, Wg, Wu, _ = make_mlp(T, H, I, "direct")
    got = run_swiglu_fused(X, Wg, Wu, offset=offset)
    gate = oracle.gemm_fp16(X, Wg)
    up = oracle.gemm_fp16(X, Wu)
    assert_swiglu_close(got, oracle.swiglu(gate, up))


def test_swiglu_fused_hidden_zero():
    out = empty_f16(3, 16, fill=float("nan"))
    dummy = to_dev(np.zeros(64, np.float16))
    _cg().swiglu_fused(dummy, dummy, dummy, out, 3, 0, 16)
    _sync()
    got = to_host(out)
    assert np.all(got == 0) and not np.any(np.signbit(got))
