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

// One workgroup per `chunk` bytes (a multiple of 4 x 32 KB), streaming its
// chunk in 32 KB steps with D steps (D x 32 KB) in flight: with few large
// chunks this measures how fast a single CU can pull data, and how that
// depends on the bytes it keeps in flight.
template <int D>
__global__ void __launch_bounds__(kThreads) stream_read_chunk(const u32x4* src, size_t chunk16, unsigned* sink) {
    constexpr size_t step = kChunk / 16;  // u32x4 per 32 KB step
    const u32x4* p = src + (size_t)blockIdx.x * chunk16;
    const size_t nsteps = chunk16 / step;
    u32x4 v[D][kLoads];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int i = 0; i < kLoads; ++i) v[d][i] = __builtin_nontemporal_load(p + d * step + (size_t)i * kThreads + threadIdx.x);
    unsigned x = 0;
    for (size_t s = 0; s < nsteps; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) x ^= v[d][i].x ^ v[d][i].y ^ v[d][i].z ^ v[d][i].w;
            const size_t t = s + d + D;  // the step this slot loads next
            if (t < nsteps) {
#pragma unroll
                for (int i = 0; i < kLoads; ++i)
                    v[d][i] = __builtin_nontemporal_load(p + t * step + (size_t)i * kThreads + threadIdx.x);
            }
        }
    }
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

// `bytes` split into bytes / chunk workgroups of `chunk` bytes each (chunk a
// multiple of 128 KB dividing bytes; src 16-byte aligned), with `depth` (1 or
// 4) steps of 32 KB in flight per workgroup.  Returns the number
// of workgroups, or -1 for bad arguments.
extern "C" int clove_diag_stream_read_chunked(const void* src, size_t bytes, size_t chunk, int depth,
                                              unsigned* sink, void* stream) {
    if (src == nullptr || sink == nullptr || chunk == 0 || chunk % (4 * kChunk) != 0 || bytes % chunk != 0 ||
        (depth != 1 && depth != 4) || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return -1;
    const size_t grid = bytes / chunk;
    if (grid == 0 || grid > 0x7fffffffu) return -1;
    auto k = depth == 4 ? stream_read_chunk<4> : stream_read_chunk<1>;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4*>(src), chunk / 16, sink);
    return hipGetLastError() == hipSuccess ? (int)grid : -1;
}
