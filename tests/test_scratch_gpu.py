"""Split-K scratch: a call that needs more scratch than its stream holds gets a
larger buffer (the old one is retired, not freed under queued work), results
stay correct before and after the growth and after clove_release_scratch()."""
import numpy as np
import pytest

import oracle
from tests._util import empty_f16, rng, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu


def _check(cg, M, N, K, key):
    import torch
    g = rng("scratch", M, N, K, key)
    A = g.standard_normal((M, K)).astype(np.float16)
    B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    C = empty_f16(M, N)
    cg.gemm_fp16(to_dev(A), to_dev(B), C, M, N, K)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 6)]))
    ref = oracle.gemm_fp16_f64(A[rows], B)
    ok, rep = within_tol(to_host(C)[rows], ref)
    assert ok, (M, N, K, key, rep)


def test_scratch_growth_and_release():
    import clove_compute_amd as cg
    print("scratch: M=32 (4 MiB of partials), then M=128 (8 MiB), then M=32 again", flush=True)
    _check(cg, 32, 4096, 4096, 0)
    _check(cg, 128, 4096, 4096, 1)
    _check(cg, 32, 4096, 4096, 2)
    cg.release_scratch()
    print("scratch: after release", flush=True)
    _check(cg, 128, 4096, 4096, 3)
    _check(cg, 32, 4096, 4096, 4)


def test_two_streams_keep_separate_scratch():
    # split-K launches on two streams at once: each stream has its own partials
    # and counters, so neither result is disturbed by the other
    import torch
    import clove_compute_amd as cg
    M, N, K = 32, 4096, 4096
    ins, outs, streams = [], [], [torch.cuda.Stream(), torch.cuda.Stream()]
    for key in range(2):
        g = rng("scratch2", key)
        A = g.standard_normal((M, K)).astype(np.float16)
        B = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
        ins.append((A, B, to_dev(A), to_dev(B)))
        outs.append(empty_f16(M, N))
    torch.cuda.synchronize()
    print("scratch: 2 streams x 4 calls", flush=True)
    for _ in range(4):
        for s, (_, _, dA, dB), C in zip(streams, ins, outs):
            with torch.cuda.stream(s):
                cg.gemm_fp16(dA, dB, C, M, N, K, stream=s)
    torch.cuda.synchronize()
    for (A, B, _, _), C in zip(ins, outs):
        rows = np.array([0, 7, 19, M - 1])
        ok, rep = within_tol(to_host(C)[rows], oracle.gemm_fp16_f64(A[rows], B))
        assert ok, rep
