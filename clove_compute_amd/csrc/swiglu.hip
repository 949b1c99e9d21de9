// SwiGLU for gfx950: out = fp16(silu(gate) * up), silu(x) = x / (1 + exp(-x))
// in fp32 -- the reference's swiglu (src/kernels/activations.cu:76-134, silu_f
// :9-11) -- and the reference's declared-but-undefined swiglu_fused
// (include/clove/kernels/activations.cuh:37-46) on FP16 weights.
//
//  * swiglu_kernel: HBM-bound elementwise pass, 16-byte loads and stores
//    (8 elements per thread), grid-stride; a scalar tail for n % 8 and for
//    unaligned pointers.
//  * swiglu_fused on FP16 weights [hidden, intermediate] (the reference's
//    gemm_fp16 B layout): gate into the output, up into a library buffer,
//    both through gemm_fp16, then SwiGLU in place.  (The INT4-weight MLP path,
//    launch_w4a16_swiglu, fuses the pair inside the GEMM instead.)
#include <algorithm>

#include "common.hpp"
#include "dispatch.hpp"

namespace clove {
namespace act {

using namespace hw;

__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t* gate,
                                                     const uint16_t* up,
                                                     uint16_t* out, int64_t n, int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t n8 = n / 8;
        for (; i < n8; i += stride) {
            const u32x4 g = reinterpret_cast<const u32x4*>(gate)[i];
            const u32x4 u = reinterpret_cast<const u32x4*>(up)[i];
            u32x4 o;
#pragma unroll
            for (int d = 0; d < 4; ++d)
                o[d] = (unsigned)swiglu_h((uint16_t)(g[d] & 0xffffu), (uint16_t)(u[d] & 0xffffu)) |
                       ((unsigned)swiglu_h((uint16_t)(g[d] >> 16), (uint16_t)(u[d] >> 16)) << 16);
            reinterpret_cast<u32x4*>(out)[i] = o;
        }
        // tail: the last n % 8 elements, one per thread of the first workgroup
        const int64_t t = n8 * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (t < n && t < n8 * 8 + 8) out[t] = swiglu_h(gate[t], up[t]);
        return;
    }
    for (; i < n; i += stride) out[i] = swiglu_h(gate[i], up[i]);
}

}  // namespace act

clove_status_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                             hipStream_t stream) {
    if (n <= 0) return CLOVE_OK;
    DeviceInfo dev;
    const clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const bool vec = aligned16(gate) && aligned16(up) && aligned16(out);
    const int64_t work = vec ? hw::cdiv64(n, 8) : n;
    // enough workgroups to keep every CU streaming, capped at 16 per CU
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(hw::cdiv64(work, 256), 16 * dev.num_cus));
    CLOVE_LAUNCH(act::swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, gate, up, out, n,
                       vec ? 1 : 0);
    return check_launch();
}

clove_status_t launch_swiglu_fused_fp16(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up,
                                        uint16_t* out, int T, int hidden, int inter, hipStream_t stream) {
    void* ubuf = nullptr;
    clove_status_t st = acquire_buffer(stream, kBufSwiglu, (size_t)T * inter * 2, &ubuf);
    if (st != CLOVE_OK) return st;
    uint16_t* u = static_cast<uint16_t*>(ubuf);
    if ((st = launch_gemm_fp16(X, W_gate, out, 1, T, inter, hidden, 1.0f, 0.0f, stream)) != CLOVE_OK) return st;
    if ((st = launch_gemm_fp16(X, W_up, u, 1, T, inter, hidden, 1.0f, 0.0f, stream)) != CLOVE_OK) return st;
    return launch_swiglu(out, u, out, (int64_t)T * inter, stream);
}

}  // namespace clove
