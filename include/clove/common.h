// Shared C++ definitions of the Clove Compute API on MI355X (HIP).
//
// Same namespace and names as the reference header include/clove/common.cuh,
// so that code written against it (its runtime, tests and bench) compiles
// unchanged apart from the CUDA runtime types: the error macros take a
// hipError_t and report through hipGetErrorString, and CLOVE_SYNC_CHECK
// synchronises the HIP device.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace clove {

// include/clove/common.cuh:11-19: print file:line and the runtime's message,
// then exit(EXIT_FAILURE).  The argument is any expression yielding a
// hipError_t (a HIP runtime call).
#define CLOVE_CHECK_HIP(call)                                                       \
    do {                                                                            \
        const hipError_t clove_err_ = (call);                                       \
        if (clove_err_ != hipSuccess) {                                             \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,    \
                         hipGetErrorString(clove_err_));                            \
            std::exit(EXIT_FAILURE);                                                \
        }                                                                           \
    } while (0)

// The reference's spelling (include/clove/common.cuh:11), kept so that its
// callers compile as written; on this platform the call is a HIP call.
#define CLOVE_CHECK_CUDA(call) CLOVE_CHECK_HIP(call)

// include/clove/common.cuh:21: the last launch error of the calling thread.
#define CLOVE_CHECK_LAST() CLOVE_CHECK_HIP(hipGetLastError())

// include/clove/common.cuh:23-27: wait for the device, then check both the
// synchronisation and the last launch.
#define CLOVE_SYNC_CHECK()                            \
    do {                                              \
        CLOVE_CHECK_HIP(hipDeviceSynchronize());      \
        CLOVE_CHECK_LAST();                           \
    } while (0)

// include/clove/common.cuh:30-32
constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// include/clove/common.cuh:35-41: element types of the runtime's tensors
enum class DType { FP32, FP16, BF16, INT8, INT4 };

// include/clove/common.cuh:43-53: bytes per element; INT4 packs two values
// per byte and reports 0, as in the reference (callers size INT4 buffers as
// numel / 2 themselves)
inline size_t dtype_size(DType dtype) {
    switch (dtype) {
        case DType::FP32: return 4;
        case DType::FP16: return 2;
        case DType::BF16: return 2;
        case DType::INT8: return 1;
        case DType::INT4: return 0;
    }
    return 0;
}

// include/clove/common.cuh:55-59: element type -> DType.  The reference's
// name is kept for source compatibility; the types are the HIP ones.
template <typename T> struct CudaType;
template <> struct CudaType<float> { using type = float; static constexpr DType dtype = DType::FP32; };
template <> struct CudaType<half> { using type = half; static constexpr DType dtype = DType::FP16; };
template <> struct CudaType<int8_t> { using type = int8_t; static constexpr DType dtype = DType::INT8; };

}  // namespace clove
