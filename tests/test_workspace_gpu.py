"""Caller-owned workspace (clove_workspace_bind / clove_workspace_query_*).

A size query plans the calls and launches nothing; with a bound workspace of
the queried size every entry point gives bit-for-bit the results it gives with
library scratch (same kernels, same split plan), allocates nothing (so it can
be captured in a HIP graph), and a call that needs more than the workspace
holds fails with CLOVE_ERR_WORKSPACE without writing its output.
"""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, f16bits, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu


def _cg():
    import clove_compute_amd as cg
    return cg


def _zeros_ws(nbytes):
    import torch
    return torch.zeros(max(nbytes, 1), dtype=torch.uint8, device="cuda")


def _fp16_case(M, N, K, key):
    g = rng("ws", M, N, K, key)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    return A, B, to_dev(A), to_dev(B)


def test_query_launches_nothing_and_sizes():
    import torch
    cg = _cg()
    _, _, dA, dB = _fp16_case(32, 4096, 4096, 0)
    C = empty_f16(32, 4096, fill=float("nan"))
    with cg.workspace_query() as q:
        cg.gemm_fp16(dA, dB, C, 32, 4096, 4096)
    torch.cuda.synchronize()
    assert q.bytes > cg.CLOVE_WORKSPACE_MIN_BYTES          # split-K partials
    assert torch.isnan(C).all().item()                       # nothing ran
    _, _, dA4, dB4 = _fp16_case(4096, 4096, 4096, 1)
    C4 = empty_f16(4096, 4096)
    with cg.workspace_query() as q4:
        cg.gemm_fp16(dA4, dB4, C4, 4096, 4096, 4096)
    assert q4.bytes == 0                                     # one tile per CU, no split
    # the largest of several calls
    with cg.workspace_query() as q2:
        cg.gemm_fp16(dA, dB, C, 32, 4096, 4096)
        cg.gemm_fp16(dA4, dB4, C4, 4096, 4096, 4096)
    assert q2.bytes == q.bytes


def test_bound_workspace_matches_library_scratch_and_rejects_overflow():
    import torch
    cg = _cg()
    A, B, dA, dB = _fp16_case(32, 4096, 4096, 2)
    ref = empty_f16(32, 4096)
    cg.gemm_fp16(dA, dB, ref, 32, 4096, 4096)
    with cg.workspace_query() as q:
        cg.gemm_fp16(dA, dB, ref, 32, 4096, 4096)
    ws = _zeros_ws(q.bytes)
    cg.workspace_bind(ws)
    try:
        for _ in range(3):  # the counters are left re-armed
            C = empty_f16(32, 4096, fill=float("nan"))
            cg.gemm_fp16(dA, dB, C, 32, 4096, 4096)
            torch.cuda.synchronize()
            assert np.array_equal(f16bits(to_host(C)), f16bits(to_host(ref)))
        # M = 128 needs more partials than this workspace holds
        A2, B2, dA2, dB2 = _fp16_case(128, 4096, 4096, 3)
        C2 = empty_f16(128, 4096, fill=float("nan"))
        with pytest.raises(cg.CloveError) as e:
            cg.gemm_fp16(dA2, dB2, C2, 128, 4096, 4096)
        assert e.value.status == cg.CLOVE_ERR_WORKSPACE
        torch.cuda.synchronize()
        assert torch.isnan(C2).all().item()
    finally:
        cg.workspace_bind()
    cg.gemm_fp16(dA2, dB2, C2, 128, 4096, 4096)  # library scratch again
    torch.cuda.synchronize()
    rows = np.array([0, 63, 127])
    ok, rep = within_tol(to_host(C2)[rows], oracle.gemm_fp16_f64(A2[rows], B2))
    assert ok, rep


def _entry_points():
    """(name, inputs, run(out) -> None, out shape) for every split-K / intermediate user."""
    import torch
    from clove_compute_amd import quant
    cg = _cg()
    g = rng("ws-all")
    cases = []
    # INT8 row/col, M = 128 (skinny split-K, int32 partials)
    A8 = to_dev(g.integers(-127, 128, (128, 4096)).astype(np.int8))
    B8 = to_dev(g.integers(-127, 128, (4096, 4096)).astype(np.int8))
    sa = to_dev(g.uniform(0.001, 0.02, 128).astype(np.float16))
    sb = to_dev(g.uniform(0.001, 0.02, 4096).astype(np.float16))
    cases.append(("int8_rowcol 128x4096x4096", (128, 4096),
                  lambda C: cg.gemm_int8_rowcol(A8, B8, sa, sb, C, 128, 4096, 4096)))
    # INT4 group-wise N = 128 (B transpose pass into the workspace, then the MFMA GEMM)
    M, N, K = 4096, 128, 4096
    G = K // 128
    Aq = to_dev(quant.pack_rows(g.integers(0, 16, (M, K))))
    Bq = to_dev(quant.pack_cols(g.integers(0, 16, (K, N))))
    sA = to_dev(g.uniform(0.001, 0.02, (M, G)).astype(np.float16))
    zA = to_dev(g.integers(0, 16, (M, G)).astype(np.float16))
    sB = to_dev(g.uniform(0.001, 0.02, (G, N)).astype(np.float16))
    zB = to_dev(g.integers(0, 16, (G, N)).astype(np.float16))
    cases.append(("int4 4096x128x4096", (M, N), lambda C: cg.gemm_int4(Aq, sA, zA, Bq, sB, zB, C, M, N, K)))
    # W4A16 T = 512 down projection with the residual (split-K MFMA GEMM)
    T, O, Kd = 512, 2048, 8192
    Gd = Kd // 128
    X = to_dev(g.standard_normal((T, Kd)).astype(np.float16))
    Wq = to_dev(quant.pack_rows(g.integers(0, 16, (O, Kd))))
    ws_ = to_dev(g.uniform(0.001, 0.02, (O, Gd)).astype(np.float16))
    wz = to_dev(g.integers(0, 16, (O, Gd)).astype(np.float16))
    Y0 = to_dev(g.standard_normal((T, O)).astype(np.float16))

    def down(C):
        C.copy_(Y0)
        cg.gemm_w4a16(X, Wq, ws_, wz, C, T, O, Kd, 1.0, 1.0)
    cases.append(("w4a16 down+res 512x2048x8192", (T, O), down))
    # FP16 swiglu_fused (an intermediate buffer and two split-K GEMMs)
    Tf, H, I = 32, 2048, 8192
    Xf = to_dev((g.standard_normal((Tf, H))).astype(np.float16))
    Wg = to_dev((g.standard_normal((H, I)) * 0.02).astype(np.float16))
    Wu = to_dev((g.standard_normal((H, I)) * 0.02).astype(np.float16))
    cases.append(("swiglu_fused fp16 32x2048x8192", (Tf, I),
                  lambda C: cg.swiglu_fused(Xf, Wg, Wu, C, Tf, H, I)))
    torch.cuda.synchronize()
    return cases


def test_every_entry_point_same_bits_with_bound_workspace():
    import torch
    cg = _cg()
    for name, shape, run in _entry_points():
        print(f"workspace: {name}", flush=True)
        ref = empty_f16(*shape)
        run(ref)
        torch.cuda.synchronize()
        with cg.workspace_query() as q:
            run(empty_f16(*shape))
        assert q.bytes > 0, name
        ws = _zeros_ws(q.bytes)
        cg.workspace_bind(ws)
        try:
            for _ in range(2):
                C = empty_f16(*shape, fill=float("nan"))
                run(C)
                torch.cuda.synchronize()
                assert np.array_equal(f16bits(to_host(C)), f16bits(to_host(ref))), name
        finally:
            cg.workspace_bind()


def test_bound_workspace_in_a_graph():
    # nothing is allocated with a bound workspace, so a split-K call can be
    # captured; every replay (with eager work between) matches the eager result
    import torch
    cg = _cg()
    A, B, dA, dB = _fp16_case(32, 4096, 4096, 5)
    ref = empty_f16(32, 4096)
    cg.gemm_fp16(dA, dB, ref, 32, 4096, 4096)
    with cg.workspace_query() as q:
        cg.gemm_fp16(dA, dB, ref, 32, 4096, 4096)
    ws = _zeros_ws(q.bytes)
    C = empty_f16(32, 4096)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    cg.workspace_bind(ws)
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            cg.gemm_fp16(dA, dB, C, 32, 4096, 4096)
        torch.cuda.synchronize()
        for i in range(3):
            C.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(f16bits(to_host(C)), f16bits(to_host(ref))), i
            _ = (dA.float() @ dA.float().T).sum().item()  # eager work between replays
    finally:
        cg.workspace_bind()
