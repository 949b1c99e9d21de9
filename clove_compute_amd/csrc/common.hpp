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
__device__ __forceinline__ uint16_t f2h(float f) {
    return bitcast<uint16_t>(static_cast<_Float16>(f));
}
__device__ __forceinline__ unsigned pack2h(float lo, float hi) {
    return static_cast<unsigned>(f2h(lo)) | (static_cast<unsigned>(f2h(hi)) << 16);
}

// ---------------------------------------------------------------------------
// split-K completion: the last workgroup of a tile to arrive reduces the
// partials.  Release/acquire at agent scope make the fp32 partials written by
// workgroups on other XCDs visible (agent-scope fences write back / invalidate
// the per-XCD L2 for coarse-grained memory).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool splitk_arrive_is_last(unsigned* counter, unsigned nsplit,
                                                      int* lds_flag) {
    __threadfence();  // release this workgroup's partial stores
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL,
                                               __HIP_MEMORY_SCOPE_AGENT);
        int last = (prev == nsplit - 1) ? 1 : 0;
        if (last) {
            // reset for the next launch on this scratch (stream order makes it safe)
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *lds_flag = last;
    }
    __syncthreads();
    const bool last = *lds_flag != 0;
    if (last) __threadfence();  // acquire the other workgroups' partials
    return last;
}

}  // namespace hw
}  // namespace clove
