// Diagnostic, not part of the GEMM C-ABI: read-only streaming kernels that
// measure the cold HBM read floor the memory-bound GEMM kernels are compared
// with, and how fast one CU pulls data by each load kind the kernels use.
// Built into lib/libclove_diag.so and used by bench.py --floor, and the shader
// clock probe (sclk_probe) bench.py runs between launches of the headline GEMM.
//
// stream_read: every workgroup reads one contiguous 32 KB chunk, 256 threads x
// 8 loads of 16 bytes, lane-contiguous (each load instruction covers 4 KB), all
// issued before the first use; the bytes are folded into one word that is
// stored only if it equals a value no input produces, so no load is dropped.
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
// depends on the bytes it keeps in flight.  Workgroup b reads from
// src + b * stride16 (stride 0: every workgroup reads the same chunk, which
// then sits in each XCD's L2); NT: nontemporal loads (the decode GEMVs'
// weight streams), else ordinary cached loads.
template <int D, bool NT>
__global__ void __launch_bounds__(kThreads) stream_read_chunk(const u32x4* src, size_t chunk16, size_t stride16,
                                                             unsigned* sink) {
    constexpr size_t step = kChunk / 16;  // u32x4 per 32 KB step
    const u32x4* p = src + (size_t)blockIdx.x * stride16;
    const size_t nsteps = chunk16 / step;
    auto ld = [&](size_t i) { return NT ? __builtin_nontemporal_load(p + i) : p[i]; };
    u32x4 v[D][kLoads];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int i = 0; i < kLoads; ++i) v[d][i] = ld(d * step + (size_t)i * kThreads + threadIdx.x);
    unsigned x = 0;
    for (size_t s = 0; s < nsteps; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) x ^= v[d][i].x ^ v[d][i].y ^ v[d][i].z ^ v[d][i].w;
            const size_t t = s + d + D;  // the step this slot loads next
            if (t < nsteps) {
#pragma unroll
                for (int i = 0; i < kLoads; ++i) v[d][i] = ld(t * step + (size_t)i * kThreads + threadIdx.x);
            }
        }
    }
    if (x == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x & 1023] = x;
}

// The same pull by LDS DMA (buffer_load_dwordx4 ... lds, the GEMM kernels'
// staging): each of the 4 waves moves 8 KB per step into its own ring of 4
// stages (128 KB of LDS), at most 3 steps behind (vmcnt); nothing reads the
// LDS, the DMAs are issued as inline asm and so are never dropped.
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14);
}
constexpr int kDmaStages = 4;
constexpr int kDmaLds = kThreads / 64 * kDmaStages * 8192;

__global__ void __launch_bounds__(kThreads) pull_dma(const unsigned char* src, unsigned chunk, size_t stride) {
    extern __shared__ unsigned char lds[];
    const unsigned lds0 = (unsigned)reinterpret_cast<uintptr_t>(lds);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const uint64_t a = reinterpret_cast<uint64_t>(src + blockIdx.x * stride);
    u32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((unsigned)a);
    r.y = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32) & 0xffffu);
    r.z = chunk;  // bytes: the hardware returns zero past them
    r.w = 0x00020000u;
    constexpr int W = kThreads / 64;
    const int nsteps = (int)(chunk / (W * 8192));
    const int voff = lane * 16 + wave * 8192;
    for (int s = 0; s < nsteps; ++s) {
        if (s >= kDmaStages) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kDmaStages - 1) * 8));
        const unsigned st = lds0 + (unsigned)(((s % kDmaStages) * W + wave) * 8192);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int soff = s * W * 8192 + i * 1024;
            // (s_nop: the wait state an LDS DMA needs after the M0 write)
            asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                         :
                         : "v"(voff), "s"(r), "s"(soff), "{m0}"(st + i * 1024)
                         : "memory");
        }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

// A second floor design: a persistent grid of `gridDim.x` workgroups of 1024
// threads, workgroup b streaming the b-th contiguous slice of the buffer in
// steps of 16 KB (one 16-byte load per thread), D steps in flight per thread
// (D x 16 KB per workgroup), lane-contiguous like the one-shot kernel.  Loads
// past the end read the last element (clamped, unconditional).
template <int D>
__global__ void __launch_bounds__(1024) stream_read_persistent(const u32x4* src, size_t n16, size_t per16,
                                                               unsigned* sink) {
    const size_t base = (size_t)blockIdx.x * per16 + threadIdx.x;
    const size_t nsteps = per16 / 1024;
    auto ld = [&](size_t s) { return __builtin_nontemporal_load(src + min(base + s * 1024, n16 - 1)); };
    u32x4 v[D];
#pragma unroll
    for (int d = 0; d < D; ++d) v[d] = ld(d);
    unsigned x = 0;
    for (size_t s = 0; s < nsteps; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            x ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
            if (s + d + D < nsteps) v[d] = ld(s + d + D);
        }
    }
    if (x == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x & 1023] = x;
}

// The shader clock: one wave reads the shader-cycle counter (s_memtime) and
// the constant 100 MHz counter (s_memrealtime), spins until the latter has
// advanced `ticks` (or `max_iters` rounds have passed, so the wave always
// ends), reads both again and stores the four values; the clock in MHz is
// 100 * (cycles after - cycles before) / (ticks after - ticks before).
__global__ void __launch_bounds__(64) sclk_probe(unsigned long long* out, unsigned ticks, unsigned max_iters) {
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    unsigned long long r1 = r0;
    for (unsigned i = 0; i < max_iters && r1 - r0 < ticks; ++i) r1 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[0] = c0;
        out[1] = r0;
        out[2] = c1;
        out[3] = r1;
    }
}

}  // namespace

// One shader-clock reading on `stream` into out[0..3] (device memory, 32
// bytes): cycles and 100 MHz ticks before and after a spin of `ticks` ticks
// (1..100000).  Returns 0, or -1 for bad arguments or a failed launch.
extern "C" int clove_diag_sclk(unsigned long long* out, unsigned ticks, void* stream) {
    if (out == nullptr || ticks == 0 || ticks > 100000) return -1;
    hipLaunchKernelGGL(sclk_probe, dim3(1), dim3(64), 0, (hipStream_t)stream, out, ticks, 1000000u);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// `bytes` (a multiple of 16, 16-byte aligned) read by `grid` persistent
// workgroups (1..4096) of 1024 threads, each over one contiguous slice, with
// `depth` (4 or 8) 16 KB steps in flight per workgroup.  Returns grid, or -1.
extern "C" int clove_diag_stream_read_persistent(const void* src, size_t bytes, int grid, int depth,
                                                 unsigned* sink, void* stream) {
    if (src == nullptr || sink == nullptr || bytes == 0 || bytes % 16 != 0 || grid <= 0 || grid > 4096 ||
        (depth != 4 && depth != 8) || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return -1;
    const size_t n16 = bytes / 16;
    const size_t per16 = (n16 + (size_t)grid * 1024 - 1) / ((size_t)grid * 1024) * 1024;  // whole 16 KB steps
    auto k = depth == 8 ? stream_read_persistent<8> : stream_read_persistent<4>;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(1024), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4*>(src), n16, per16, sink);
    return hipGetLastError() == hipSuccess ? grid : -1;
}

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
// 4) steps of 32 KB in flight per workgroup, nontemporal loads.  Returns the
// number of workgroups, or -1 for bad arguments.
extern "C" int clove_diag_stream_read_chunked(const void* src, size_t bytes, size_t chunk, int depth,
                                              unsigned* sink, void* stream) {
    if (src == nullptr || sink == nullptr || chunk == 0 || chunk % (4 * kChunk) != 0 || bytes % chunk != 0 ||
        (depth != 1 && depth != 4) || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return -1;
    const size_t grid = bytes / chunk;
    if (grid == 0 || grid > 0x7fffffffu) return -1;
    auto k = depth == 4 ? stream_read_chunk<4, true> : stream_read_chunk<1, true>;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4*>(src), chunk / 16, chunk / 16, sink);
    return hipGetLastError() == hipSuccess ? (int)grid : -1;
}

// One workgroup's pull rate by load kind: `grid` workgroups of 256 threads
// each read `chunk` bytes (a multiple of 128 KB, below 2 GiB), workgroup b at
// src + b * chunk, or all of them at src when `shared` (the chunk is then L2
// resident).  kind 0: nontemporal loads, 1: ordinary loads (4 x 32 KB in
// flight), 2: LDS DMA (4 stages of 32 KB).  src must hold grid x chunk bytes
// (chunk when shared) and be 16-byte aligned.  Returns grid, or -1.
extern "C" int clove_diag_pull(const void* src, size_t chunk, int grid, int shared, int kind, unsigned* sink,
                               void* stream) {
    if (src == nullptr || sink == nullptr || chunk == 0 || chunk % (4 * kChunk) != 0 ||
        chunk >= ((size_t)1 << 31) || grid <= 0 || grid > 65536 || kind < 0 || kind > 2 ||
        (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return -1;
    const size_t stride = shared ? 0 : chunk;
    hipStream_t s = (hipStream_t)stream;
    if (kind == 2) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(pull_dma),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kDmaLds) != hipSuccess)
            return -1;
        hipLaunchKernelGGL(pull_dma, dim3((unsigned)grid), dim3(kThreads), kDmaLds, s,
                           reinterpret_cast<const unsigned char*>(src), (unsigned)chunk, stride);
    } else {
        auto k = kind == 0 ? stream_read_chunk<4, true> : stream_read_chunk<4, false>;
        hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kThreads), 0, s, reinterpret_cast<const u32x4*>(src),
                           chunk / 16, stride / 16, sink);
    }
    return hipGetLastError() == hipSuccess ? grid : -1;
}
