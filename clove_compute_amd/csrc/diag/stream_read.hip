// Diagnostic, not part of the GEMM C-ABI: a read-only streaming kernel that
// measures the cold HBM read floor the memory-bound GEMM kernels are compared
// with.  Built into lib/libclove_diag.so and used by bench.py --floor only.
//
// Every workgroup reads one contiguous 32 KB chunk: 256 threads x 8 loads of
// 16 bytes, lane-contiguous (each load instruction covers 4 KB), all issued
// before the first use; the bytes are folded into one word that is stored
// only if it equals a value no input produces, so no load is dropped.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256, kLoads = 8, kChunk = kThreads * kLoads * 16;

__global__ void __launch_bounds__(kThreads) stream_read(const u32x4* src, size_t n16, unsigned* sink) {
    const size_t base = (size_t)blockIdx.x * (kChunk / 16) + threadIdx.x;
    u32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const size_t j = base + (size_t)i * kThreads;
        v[i] = j < n16 ? __builtin_nontemporal_load(src + j) : u32x4{0u, 0u, 0u, 0u};
    }
    unsigned x = 0;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x & 1023] = x;
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) at src on `stream`.
// Returns the number of workgroups launched, or -1 for bad arguments.
extern "C" int clove_diag_stream_read(const void* src, size_t bytes, unsigned* sink, void* stream) {
    if (src == nullptr || sink == nullptr || bytes == 0 || bytes % 16 != 0 ||
        (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return -1;
    const size_t grid = (bytes + kChunk - 1) / kChunk;
    if (grid > 0x7fffffffu) return -1;
    hipLaunchKernelGGL(stream_read, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4*>(src), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? (int)grid : -1;
}
