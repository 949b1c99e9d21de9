// Shared device/host definitions for the gfx950 GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace clove {
namespace hw {

// ---------------------------------------------------------------------------
// vector types (clang ext_vector_type: map 1:1 onto VGPR tuples)
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;           // CDNA wavefront
constexpr int kGroup = 128;         // INT4 quantisation group along K

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From& v) {
    static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
    return __builtin_bit_cast(To, v);
}

// fp16 <-> fp32 (hardware conversions; narrowing is round-to-nearest-even in
// the default MODE register)
__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(bitcast<_Float16>(h));
}
// The empty asm pins f as an fp32 register value: without it the backend folds
// a preceding fp32 multiply into the narrowing (v_fma_mixlo_f16, one rounding
// of the exact product), while the reference rounds to fp32 first and then to
// fp16 (float result = ...; __float2half(result)).
__device__ __forceinline__ uint16_t f2h(float f) {
    asm("" : "+v"(f));
    return bitcast<uint16_t>(static_cast<_Float16>(f));
}
__device__ __forceinline__ unsigned pack2h(float lo, float hi) {
    return static_cast<unsigned>(f2h(lo)) | (static_cast<unsigned>(f2h(hi)) << 16);
}

// SwiGLU of one fp16 gate / up pair: fp16(silu(g) * u), silu(x) = x / (1 +
// exp(-x)) in fp32 (src/kernels/activations.cu:9-11, :76-134); expf is the
// device library's, the division IEEE fp32
__device__ __forceinline__ uint16_t swiglu_h(uint16_t g, uint16_t u) {
    const float x = h2f(g);
    const float s = x / (1.0f + expf(-x));
    return f2h(s * h2f(u));
}

// ---------------------------------------------------------------------------
// Cross-lane sums without the LDS pipe: gfx950's v_permlane16_swap /
// v_permlane32_swap exchange 16-lane rows (or 32-lane halves) between two
// registers in the VALU.  With the rows of a wave r0..r3:
//   permlane16_swap(x, y) -> {[x0 y0 x2 y2], [x1 y1 x3 y3]}
//   permlane32_swap(x, y) -> {[x0 x1 y0 y1], [x2 x3 y2 y3]}
// so adding the two results sums two registers across the swapped lanes at
// once, each in its own half of the wave.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T swap_sum16(T x, T y) {
    const auto s = __builtin_amdgcn_permlane16_swap(bitcast<unsigned>(x), bitcast<unsigned>(y), false, false);
    return bitcast<T>(s[0]) + bitcast<T>(s[1]);
}
template <typename T>
__device__ __forceinline__ T swap_sum32(T x, T y) {
    const auto s = __builtin_amdgcn_permlane32_swap(bitcast<unsigned>(x), bitcast<unsigned>(y), false, false);
    return bitcast<T>(s[0]) + bitcast<T>(s[1]);
}
// Four registers summed over the four lanes l, l^16, l^32, l^48: lane l of
// row r returns the sum of v[r], added as (row 0 + row 1) + (row 2 + row 3)
// -- the order of an xor-16 then xor-32 butterfly.
template <typename T>
__device__ __forceinline__ T rows_sum4(T v0, T v1, T v2, T v3) {
    return swap_sum32(swap_sum16(v0, v1), swap_sum16(v2, v3));
}
// Two registers summed over lanes l and l^32: lanes 0..31 return the sum of
// x, lanes 32..63 that of y, each as (lane l) + (lane l + 32).
template <typename T>
__device__ __forceinline__ T halves_sum2(T x, T y) {
    return swap_sum32(x, y);
}

// One register summed over all 64 lanes, every lane returning the total,
// without the LDS pipe: inside each 16-lane row DPP row_ror:8 (lane l ^ 8),
// row_ror:4 (with the step before, the 4 lanes of l's class mod 4) and the
// quad_perm swaps [2,3,0,1] (l ^ 2) and [1,0,3,2] (l ^ 1) leave the row's
// sum in every lane of the row; the four row sums are read into scalars and
// added as (row 0 + row 1) + (row 2 + row 3).  A fixed order (the same bits
// on every call), and one extra register per value.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    v = v + bitcast<T>(__builtin_amdgcn_mov_dpp(bitcast<int>(v), 0x128, 0xf, 0xf, false));  // row_ror:8
    v = v + bitcast<T>(__builtin_amdgcn_mov_dpp(bitcast<int>(v), 0x124, 0xf, 0xf, false));  // row_ror:4
    v = v + bitcast<T>(__builtin_amdgcn_mov_dpp(bitcast<int>(v), 0x4e, 0xf, 0xf, false));   // quad_perm 2301
    v = v + bitcast<T>(__builtin_amdgcn_mov_dpp(bitcast<int>(v), 0xb1, 0xf, 0xf, false));   // quad_perm 1032
    const T r0 = bitcast<T>(__builtin_amdgcn_readlane(bitcast<int>(v), 0));
    const T r1 = bitcast<T>(__builtin_amdgcn_readlane(bitcast<int>(v), 16));
    const T r2 = bitcast<T>(__builtin_amdgcn_readlane(bitcast<int>(v), 32));
    const T r3 = bitcast<T>(__builtin_amdgcn_readlane(bitcast<int>(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Streaming GEMVs with V weight columns (or token rows): the wide variants
// (V >= WIDE) and the byte-gathering unaligned ones need more than the 128
// VGPRs a 1024-thread workgroup leaves, so they run with at most 512 threads
// (256 VGPRs).
template <int V, bool ALIGNED, int WIDE>
__host__ __device__ constexpr int gemv_max_threads() {
    return (V >= WIDE || !ALIGNED) ? 512 : 1024;
}

// ---------------------------------------------------------------------------
// Workgroup barrier for an LDS hand-off only: waits for this wave's LDS
// operations (lgkmcnt) but not for its global loads still in flight, which
// __syncthreads() would (its workgroup fence waits on vmcnt(0)).  The empty
// asm statements keep the compiler from moving LDS accesses across it.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt unconstrained
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// split-K publication without whole-cache maintenance.
//
// Partials are written with agent-scope relaxed atomic stores (global_store
// ... sc1: written through past the per-XCD L2) and read back with agent-scope
// relaxed atomic loads (sc1: served from the device-coherent level), so no
// L2 writeback/invalidate (what __threadfence() costs on a multi-XCD part) is
// needed.  Each thread waits for its own stores to be acknowledged before the
// workgroup barrier; thread 0 then bumps the tile's counter.  The workgroup
// that observes count == nsplit-1 is the last one and reduces.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool splitk_arrive_is_last(unsigned* counter, unsigned nsplit,
                                                      int* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's coherent stores are acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = (prev == nsplit - 1) ? 1 : 0;
        // the last arriver re-arms the counter for the next launch on this scratch
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// ---------------------------------------------------------------------------
// Split-K partial tiles, 16 bytes per access.  A split's slab holds NC chunks
// of 16 bytes per thread, laid out [chunk][thread] so that every chunk is one
// contiguous row of NT x 16 bytes.  Stores and loads carry cache policy sc1
// (device-coherent: written through past the XCD-private L2, read from the
// coherent level) and go through compiler builtins, never inline asm: the
// backend must see a store to keep its data registers intact until the
// hardware has read them.  The sum runs in split order (deterministic).
// ---------------------------------------------------------------------------
constexpr int kCpolSc1 = 16;

template <int NC, int NT>
__device__ __forceinline__ void splitk_publish(float* slab, int tid, const f32x4 (&v)[NC]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(slab, (short)0, NC * NT * 16, 0x00020000);
#pragma unroll
    for (int c = 0; c < NC; ++c)
        __builtin_amdgcn_raw_buffer_store_b128(bitcast<u32x4>(v[c]), r, (c * NT + tid) * 16, 0, kCpolSc1);
}

// slabs: the nsplit consecutive slabs of one tile; INT sums int32 lanes.
// `sum` holds the caller's own partial (the one it published as split `own`)
// on entry and the total on return; the own slab is not read back (SKIP_OWN,
// for up to 32 chunks per thread: beyond that the copy of the own partial
// would not fit the registers of the kernels that use it).
// Chunks are reduced 16 at a time (bounded registers); within a chunk group
// the loads of SB splits (up to 32 loads) are in flight together, so a small
// tile needs one round trip to the coherent level for all of its splits.
template <int NC, int NT, bool INT, bool SKIP_OWN = (NC <= 32)>
__device__ __forceinline__ void splitk_reduce(const float* slabs, int nsplit, int own, int tid, f32x4 (&sum)[NC]) {
    constexpr int CG = NC < 16 ? NC : 16;
    constexpr int SB = 32 / CG > 1 ? 32 / CG : 1;
    static_assert(NC % CG == 0, "chunk groups");
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(slabs), (short)0, nsplit * NC * NT * 16, 0x00020000);
#pragma unroll
    for (int c0 = 0; c0 < NC; c0 += CG) {
        f32x4 mine[SKIP_OWN ? CG : 1];
        if constexpr (SKIP_OWN) {
#pragma unroll
            for (int c = 0; c < CG; ++c) mine[c] = sum[c0 + c];
        }
        for (int s0 = 0; s0 < nsplit; s0 += SB) {
            f32x4 buf[SB][CG];
#pragma unroll
            for (int b = 0; b < SB; ++b) {
                if (s0 + b >= nsplit) break;  // uniform: no loads past the last split
                if constexpr (SKIP_OWN) {
                    if (s0 + b == own) {  // uniform: the own partial is in registers
#pragma unroll
                        for (int c = 0; c < CG; ++c) buf[b][c] = mine[c];
                        continue;
                    }
                }
#pragma unroll
                for (int c = 0; c < CG; ++c)
                    buf[b][c] = bitcast<f32x4>(__builtin_amdgcn_raw_buffer_load_b128(
                        r, (((s0 + b) * NC + c0 + c) * NT + tid) * 16, 0, kCpolSc1));
            }
#pragma unroll
            for (int b = 0; b < SB; ++b) {
                if (s0 + b >= nsplit) break;
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    if (s0 + b == 0) sum[c0 + c] = buf[b][c];
                    else if constexpr (INT)
                        sum[c0 + c] = bitcast<f32x4>(bitcast<i32x4>(sum[c0 + c]) + bitcast<i32x4>(buf[b][c]));
                    else sum[c0 + c] += buf[b][c];
                }
            }
        }
    }
}

}  // namespace hw
}  // namespace clove
