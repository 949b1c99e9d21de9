"""GPU parity of the whole W4A16 decoder-layer GEMM chain, each step fed with
the previous step's device output, against the oracle run as the same chain.

The chain is the linear part of LlamaInference::transformer_layer
(src/runtime/inference.cu:139-194) on INT4 weights, hidden 2048, intermediate
8192, with the attention and the norms (out of scope) left out:

    q    = X  @ Wqkv^T                        (QKV, 2048 -> 3072)
    res1 = Attn @ Wo^T + res0                 (O with the beta = 1 residual)
    gate = res1 @ Wg^T,  up = res1 @ Wu^T     (2048 -> 8192)
    h    = swiglu(gate, up)
    out  = h @ Wd^T + res1                    (down with the beta = 1 residual)

Attn stands for the attention output (a separate input).  Every device step
is checked against the oracle on the inputs it was given (the previous device
output) to the W4A16 tolerance, and the device chain's output against the
oracle run as the same chain on its own fp16 steps (normwise, and elementwise
away from zero).  Token rows are independent, so the oracle runs on a sample
of rows of the T = 512 batch.  The same chain with the fused gate / up +
SwiGLU (clove_w4a16_swiglu on the [gate; up] weight) is held to the same
checks.
"""
import numpy as np
import pytest

import oracle
from tests._util import rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu

HID, INTER = 2048, 8192


def _weights(key):
    from clove_compute_amd import quant
    g = rng("chain-w", key)
    out = {}
    for name, O, K in (("qkv", 3072, HID), ("o", HID, HID), ("gate", INTER, HID), ("up", INTER, HID),
                       ("down", HID, INTER)):
        G = K // 128
        q = g.integers(0, 16, (O, K))
        s = g.uniform(0.001, 0.02, (O, G)).astype(np.float16)
        z = g.integers(0, 16, (O, G)).astype(np.float16)
        out[name] = (quant.pack_rows(q), s, z)
    return out


@pytest.mark.parametrize("T", [1, 3, 24, 512])
def test_w4a16_layer_chain(T):
    import torch
    import clove_compute_amd as cg
    print(f"layer chain T={T}", flush=True)
    W = _weights("layer")
    g = rng("chain-x", T)
    X = g.standard_normal((T, HID)).astype(np.float16)
    Attn = g.standard_normal((T, HID)).astype(np.float16)
    # activations after a norm are O(1); the residual stream is kept the same scale
    res0 = g.standard_normal((T, HID)).astype(np.float16)

    dW = {k: tuple(to_dev(a) for a in v) for k, v in W.items()}
    dX, dAttn = to_dev(X), to_dev(Attn)
    q = torch.empty(T, 3072, dtype=torch.float16, device="cuda")
    res = to_dev(res0)
    gate = torch.empty(T, INTER, dtype=torch.float16, device="cuda")
    up = torch.empty_like(gate)
    h = torch.empty_like(gate)
    cg.gemm_w4a16(dX, *dW["qkv"], q, T, 3072, HID, 1.0, 0.0)
    cg.gemm_w4a16(dAttn, *dW["o"], res, T, HID, HID, 1.0, 1.0)
    res1 = res.clone()
    cg.gemm_w4a16(res1, *dW["gate"], gate, T, INTER, HID, 1.0, 0.0)
    cg.gemm_w4a16(res1, *dW["up"], up, T, INTER, HID, 1.0, 0.0)
    cg.swiglu(gate, up, h, T * INTER)
    cg.gemm_w4a16(h, *dW["down"], res, T, HID, INTER, 1.0, 1.0)

    # the same chain with the fused gate / up + SwiGLU on the stacked weight
    Wgu = tuple(to_dev(np.concatenate([W["gate"][i], W["up"][i]], 0)) for i in range(3))
    h_f = torch.empty_like(gate)
    res_f = res1.clone()
    cg.w4a16_swiglu(res1, *Wgu, h_f, T, INTER, HID)
    cg.gemm_w4a16(h_f, *dW["down"], res_f, T, HID, INTER, 1.0, 1.0)
    torch.cuda.synchronize()

    rows = np.arange(T) if T <= 24 else np.unique(np.concatenate([[0, T - 1], g.integers(0, T, 6)]))
    q_g, r1_g, gate_g, up_g, h_g, out_g = (to_host(t)[rows] for t in (q, res1, gate, up, h, res))
    hf_g, outf_g = to_host(h_f)[rows], to_host(res_f)[rows]

    # step by step: every step against the oracle on the inputs the device step
    # was given (the previous device output), to the W4A16 tolerance
    steps = [("qkv", q_g, oracle.w4a16(X[rows], *W["qkv"])[1]),
             ("o+res", r1_g, oracle.w4a16(Attn[rows], *W["o"], res0[rows], 1.0, 1.0)[1]),
             ("gate", gate_g, oracle.w4a16(r1_g, *W["gate"])[1]),
             ("up", up_g, oracle.w4a16(r1_g, *W["up"])[1]),
             ("swiglu", h_g, oracle.swiglu(gate_g, up_g).astype(np.float64)),
             ("down+res", out_g, oracle.w4a16(h_g, *W["down"], r1_g, 1.0, 1.0)[1]),
             ("fused gate/up+swiglu", hf_g, oracle.w4a16_swiglu(r1_g, *(np.concatenate([W["gate"][i], W["up"][i]], 0)
                                                                         for i in range(3))).astype(np.float64)),
             ("fused down+res", outf_g, oracle.w4a16(hf_g, *W["down"], r1_g, 1.0, 1.0)[1])]
    for name, got, ref in steps:
        ok, rep = within_tol(got, ref)
        assert ok, (T, name, rep)

    # end to end: the oracle run as the same chain on its own fp16 steps.  The
    # two chains round their intermediates independently (h near 40, one fp16
    # ulp 0.03), and those roundings move the 8192-term down sums by more than
    # the floored elementwise bound allows near zero, so this comparison is
    # normwise, and elementwise away from zero
    r1_o, _ = oracle.w4a16(Attn[rows], *W["o"], res0[rows], 1.0, 1.0)
    h_o = oracle.swiglu(oracle.w4a16(r1_o, *W["gate"])[0], oracle.w4a16(r1_o, *W["up"])[0])
    _, out64 = oracle.w4a16(h_o, *W["down"], r1_o, 1.0, 1.0)
    rms = float(np.sqrt(np.mean(out64 ** 2)))
    big = np.abs(out64) >= 0.1 * rms
    for name, got in (("chain", out_g), ("fused chain", outf_g)):
        err = np.abs(got.astype(np.float64) - out64)
        assert np.max(err) <= 2e-3 * np.max(np.abs(out64)), (T, name, float(np.max(err)))
        assert np.all(err[big] <= 1e-2 * np.abs(out64[big])), (T, name)
