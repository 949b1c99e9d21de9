"""clove_gemm_fp16_noalloc, the FP16 entry point that allocates nothing,
against clove_gemm_fp16 through the C ABI.

The two run the same kernels with the same split plans, so their outputs are
compared bit for bit: two calls in a row (the second smaller, reusing the
fixed array and its re-armed counters), then the first shape again.  A call
whose split-K scratch exceeds CLOVE_NOALLOC_SCRATCH_BYTES is rejected before
anything is launched (and a size query reports it the same way), the
documented domain (M <= 512, N, K <= 8192, aligned, N % 8 == 0, K % 64 == 0)
is checked with the library's own size query, and a first call on a fresh
stream is captured into a HIP graph and replayed against the eager output.
"""
import ctypes

import numpy as np
import pytest

from tests._util import empty_f16, f16bits, rng, to_dev, to_host

pytestmark = pytest.mark.gpu


def _abi(name, A, B, C, M, N, K, alpha=1.0, beta=0.0):
    import torch
    from clove_compute_amd import _lib
    fn = getattr(_lib.lib(), name)
    return fn(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, alpha, beta,
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _run_pair(M, N, K, key, beta):
    import torch
    g = rng("noalloc", key, M, N, K)
    A = to_dev(g.standard_normal((M, K)).astype(np.float16))
    B = to_dev((g.standard_normal((K, N)) * 0.05).astype(np.float16))
    C0 = g.standard_normal((M, N)).astype(np.float16)
    C_ref, C_na = to_dev(C0), to_dev(C0)
    assert _abi("clove_gemm_fp16", A, B, C_ref, M, N, K, 0.75, beta) == 0
    assert _abi("clove_gemm_fp16_noalloc", A, B, C_na, M, N, K, 0.75, beta) == 0
    torch.cuda.synchronize()
    return to_host(C_ref), to_host(C_na)


def test_noalloc_equals_gemm_fp16_two_calls():
    # split-K on the skinny kernel, then a smaller call on the split-K GEMV,
    # then the first shape again; every output bit for bit
    for (M, N, K), beta in (((128, 4096, 4096), 0.5), ((2, 1024, 2048), 0.0), ((128, 4096, 4096), 0.0)):
        ref, got = _run_pair(M, N, K, "pair", beta)
        assert np.array_equal(f16bits(got), f16bits(ref)), (M, N, K)
        assert np.all(np.isfinite(got.astype(np.float32)))


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (32, 4096, 4096), (512, 4096, 4096), (300, 1000, 640),
                                   (77, 45, 131), (4096, 4096, 4096), (2048, 4096, 8192), (1900, 4000, 8256)])
def test_noalloc_shapes(M, N, K):
    # the GEMV, skinny, mid-size, generic (unaligned) and 256x256 kernels, and
    # the 256x256 kernel's K split (its 64 MiB of partials in the fixed array)
    ref, got = _run_pair(M, N, K, "shapes", 0.25)
    assert np.array_equal(f16bits(got), f16bits(ref))


def _query_need(M, N, K, A, B, C):
    from clove_compute_amd import _lib
    L = _lib.lib()
    assert L.clove_workspace_query_begin() == 0
    st = _abi("clove_gemm_fp16", A, B, C, M, N, K)
    need = L.clove_workspace_query_end()
    assert st == 0
    return need


def test_noalloc_rejects_calls_beyond_its_array():
    import torch
    import clove_compute_amd as cg
    M, N, K = 4, 36864, 32768  # GEMV partials: 144 column blocks x 128 splits x 4 rows x 1 KB (72 MiB)
    A = empty_f16(M, K)
    B = torch.zeros(K, N, dtype=torch.float16, device="cuda")
    C = empty_f16(M, N, fill=float("nan"))
    assert _query_need(M, N, K, A, B, C) > cg.CLOVE_NOALLOC_SCRATCH_BYTES
    assert _abi("clove_gemm_fp16_noalloc", A, B, C, M, N, K) == cg.CLOVE_ERR_SCRATCH_LIMIT
    torch.cuda.synchronize()
    assert np.all(np.isnan(to_host(C).astype(np.float32)))  # nothing was launched
    # the entry point still works afterwards
    ref, got = _run_pair(64, 512, 1024, "after", 0.0)
    assert np.array_equal(f16bits(got), f16bits(ref))


def test_noalloc_documented_domain_fits():
    import torch
    import clove_compute_amd as cg
    A = empty_f16(512, 8192)
    B = empty_f16(8192, 8192)
    C = empty_f16(512, 8192)
    worst = 0
    for M in (1, 2, 3, 4, 5, 16, 32, 33, 64, 65, 100, 128, 129, 200, 256, 257, 300, 511, 512):
        for N in (8, 64, 136, 1000, 4096, 8192):
            for K in (64, 512, 4096, 8192):
                worst = max(worst, _query_need(M, N, K, A, B, C))
    assert 0 < worst <= cg.CLOVE_NOALLOC_SCRATCH_BYTES, worst
    big = torch.empty(4096, 4096, dtype=torch.float16, device="cuda")
    assert _query_need(4096, 4096, 4096, big, big.clone(), big.clone()) == 0


def test_noalloc_in_a_size_query():
    # inside a query the entry point plans like the real call: a call beyond
    # the array is reported as CLOVE_ERR_SCRATCH_LIMIT, one that fits as OK,
    # and the query's size is not changed by either
    import torch
    import clove_compute_amd as cg
    from clove_compute_amd import _lib
    L = _lib.lib()
    A = empty_f16(4, 32768)
    B = torch.zeros(32768, 36864, dtype=torch.float16, device="cuda")
    C = empty_f16(4, 36864, fill=float("nan"))
    A2, B2, C2 = empty_f16(128, 4096), empty_f16(4096, 4096), empty_f16(128, 4096)
    assert L.clove_workspace_query_begin() == 0
    big = _abi("clove_gemm_fp16_noalloc", A, B, C, 4, 36864, 32768)
    fits = _abi("clove_gemm_fp16_noalloc", A2, B2, C2, 128, 4096, 4096)
    need = L.clove_workspace_query_end()
    assert big == cg.CLOVE_ERR_SCRATCH_LIMIT
    assert fits == 0
    assert need == 0
    torch.cuda.synchronize()
    assert np.all(np.isnan(to_host(C).astype(np.float32)))  # a query launches nothing


@pytest.mark.parametrize("M,N,K", [(128, 4096, 4096), (2, 1024, 2048)])
def test_noalloc_first_call_on_a_fresh_stream_captured(M, N, K):
    # the split-K skinny kernel and the split-K GEMV: the first call on a new
    # stream is captured into a HIP graph (nothing to allocate), replayed three
    # times with eager work and synchronisation between the replays, and every
    # replay's output equals the eager call's bit for bit
    import torch
    g = rng("noalloc-graph", M, N, K)
    A = to_dev(g.standard_normal((M, K)).astype(np.float16))
    B = to_dev((g.standard_normal((K, N)) * 0.05).astype(np.float16))
    C_eager = empty_f16(M, N)
    assert _abi("clove_gemm_fp16_noalloc", A, B, C_eager, M, N, K) == 0
    torch.cuda.synchronize()
    ref = to_host(C_eager)
    C = empty_f16(M, N)
    # operands of the eager call made between the replays (64 x 512 x 1024)
    X2 = torch.ones(64, 1024, dtype=torch.float16, device="cuda")
    W2 = torch.full((1024, 512), 0.5, dtype=torch.float16, device="cuda")
    O2 = empty_f16(64, 512)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        st = _abi("clove_gemm_fp16_noalloc", A, B, C, M, N, K)
    assert st == 0
    for i in range(3):
        C.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(f16bits(to_host(C)), f16bits(ref)), i
        # eager work between replays, on the same array
        assert _abi("clove_gemm_fp16_noalloc", X2, W2, O2, 64, 512, 1024) == 0
        torch.cuda.synchronize()
        assert torch.all(O2 == 512.0)
    del graph
