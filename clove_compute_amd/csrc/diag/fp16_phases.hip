// Phase timestamps of the FP16 256x256 LDS-DMA GEMM (dma::gemm_f16_big_ts,
// f16_dma_gemm.hpp): the product kernel's body with a shader-cycle and a
// 100 MHz timestamp at its phase boundaries, one record per workgroup.
// Used by bench.py --phases for the headline's per-phase breakdown; not part
// of the GEMM C-ABI.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "f16_dma_gemm.hpp"

using namespace clove;

// C = A @ B (alpha 1, beta 0) on `stream` with the timestamps in `ts`
// (dma::kTsWords 64-bit words per workgroup, grid = ceil(M/256) * ceil(N/256)
// workgroups).  The operands must meet the product kernel's conditions
// (16-byte aligned, K % 64 == 0, N % 8 == 0, each operand < 2^31 bytes).
// Returns the number of workgroups launched, or -1.
extern "C" int clove_diag_fp16_big_phases(const void* A, const void* B, void* C, int M, int N, int K,
                                          unsigned long long* ts, void* stream) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!A || !B || !C || !ts || M < 1 || N < 8 || K < 64 || K % 64 != 0 || N % 8 != 0 || !al(A) || !al(B) ||
        !al(C) || (int64_t)M * K * 2 >= (1ll << 31) || (int64_t)K * N * 2 >= (1ll << 31) ||
        (int64_t)M * N * 2 >= (1ll << 31))
        return -1;
    dma::Args a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C),
                M, N, K, 1.0f, 0.0f, (int64_t)M * K, (int64_t)K * N, (int64_t)M * N,
                (M + dma::Big::BM - 1) / dma::Big::BM, (N + dma::Big::BN - 1) / dma::Big::BN};
    const int grid = a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL(dma::gemm_f16_big_ts<dma::Big>, dim3((unsigned)grid), dim3(dma::Big::NT), 0,
                       (hipStream_t)stream, a, ts);
    return hipGetLastError() == hipSuccess ? grid : -1;
}
