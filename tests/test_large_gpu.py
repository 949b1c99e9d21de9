"""Operands past 2^31 bytes: the decode paths index with 64-bit offsets.

The reference indexes with int (A[globalM*K+globalK], src/kernels/gemm_fp16.cu:88),
which wraps past 2^31 elements; the library keeps public dimensions int and
computes every global offset in 64 bits.  Each case builds one operand just over
2 GiB on the GPU (torch's generator, seeded), runs the entry point, and checks
sampled outputs against the oracle on the sampled rows / columns copied back.
"""
import numpy as np
import pytest

import oracle
from tests._util import f16bits, to_dev, to_host, within_tol

pytestmark = pytest.mark.gpu

TWO_GIB = 2 ** 31


def _gen(seed):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def test_fp16_decode_weights_over_2gib():
    import torch
    import clove_compute_amd as cg
    M, N, K = 1, 65536, 16400
    assert K * N * 2 > TWO_GIB
    print(f"large fp16 gemv: B {K}x{N} fp16 ({K * N * 2 / 2**30:.2f} GiB)", flush=True)
    g = _gen(1)
    B = (torch.randn((K, N), generator=g, device="cuda", dtype=torch.float32) * 0.02).half()
    A = torch.randn((M, K), generator=g, device="cuda", dtype=torch.float32).half()
    C = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    cg.gemm_fp16(A, B, C, M, N, K)
    torch.cuda.synchronize()
    cols = np.array([0, 1, 4095, 40000, N - 2, N - 1])
    Bc = to_host(B[:, torch.as_tensor(cols, device="cuda")].contiguous())
    ref = oracle.gemm_fp16_f64(to_host(A), Bc)
    ok, rep = within_tol(to_host(C)[:, cols], ref)
    assert ok, rep
    assert not torch.isnan(C).any().item()
    del B


def test_int8_decode_weights_over_2gib():
    import torch
    import clove_compute_amd as cg
    M, N, K = 1, 65536, 32784
    assert K * N > TWO_GIB
    print(f"large int8 gemv: B {K}x{N} int8 ({K * N / 2**30:.2f} GiB)", flush=True)
    g = _gen(2)
    B = torch.randint(-127, 128, (K, N), generator=g, device="cuda", dtype=torch.int8)
    A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    C = torch.empty((M, N), dtype=torch.float16, device="cuda")
    cg.gemm_int8(A, B, C, M, N, K, 0.01, 0, 0.02, 0)
    torch.cuda.synchronize()
    cols = np.array([0, 15, 16, 33333, N - 1])
    Bc = B[:, torch.as_tensor(cols, device="cuda")].contiguous().cpu().numpy()
    Cref, _ = oracle.gemm_int8(A.cpu().numpy(), Bc, 0.01, 0, 0.02, 0)
    assert np.array_equal(f16bits(to_host(C)[:, cols]), f16bits(Cref))
    del B


def test_int4_decode_weights_over_2gib():
    import torch
    import clove_compute_amd as cg
    M, N, K = 131200, 1, 32768
    G = K // 128
    assert M * (K // 2) > TWO_GIB
    print(f"large int4 gemv: A_q {M}x{K // 2} bytes ({M * K / 2 / 2**30:.2f} GiB)", flush=True)
    g = _gen(3)
    Aq = torch.randint(0, 256, (M, K // 2), generator=g, device="cuda", dtype=torch.uint8)
    sA = (torch.rand((M, G), generator=g, device="cuda") * 0.019 + 0.001).half()
    zA = torch.randint(0, 16, (M, G), generator=g, device="cuda").half()
    rng = np.random.default_rng(4)
    Bq = rng.integers(0, 256, (K, 1)).astype(np.uint8) & 0xF0  # N = 1: column 0 in the high nibble
    sB = rng.uniform(0.001, 0.02, (G, 1)).astype(np.float16)
    zB = rng.integers(0, 16, (G, 1)).astype(np.float16)
    C = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    cg.gemm_int4(Aq, sA, zA, to_dev(Bq), to_dev(sB), to_dev(zB), C, M, N, K)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 65535, 65536, 100000, M - 1])
    ri = torch.as_tensor(rows, device="cuda")
    _, ref, _ = oracle.gemm_int4_groupwise(Aq[ri].cpu().numpy(), to_host(sA[ri]), to_host(zA[ri]), Bq, sB, zB,
                                           len(rows), N, K)
    ok, rep = within_tol(to_host(C)[rows], ref)
    assert ok, rep
    assert not torch.isnan(C).any().item()
    del Aq
