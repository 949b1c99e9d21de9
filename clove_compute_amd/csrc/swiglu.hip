// SwiGLU for gfx950: out = fp16(silu(gate) * up), silu(x) = x / (1 + exp(-x))
// in fp32 -- the reference's swiglu (src/kernels/activations.cu:76-134, silu_f
// :9-11) -- and the reference's declared-but-undefined swiglu_fused
// (include/clove/kernels/activations.cuh:37-46) on FP16 weights.
//
//  * swiglu_kernel: HBM-bound elementwise pass, 16-byte loads and stores
//    (8 elements per thread), grid-stride; a scalar tail for n % 8 and for
//    unaligned pointers.
//  * swiglu_fused on FP16 weights [hidden, intermediate] (the reference's
//    gemm_fp16 B layout), one launch that writes neither projection to
//    memory: the FP16 GEMV with two weight operands for T <= 4, the skinny
//    MFMA kernel with two B operands for T > 4 and for T = 2..4 on large
//    weights, as gemm_fp16 decides per projection (both bit-identical to two
//    gemm_fp16 calls followed by swiglu on the shapes where gemm_fp16 takes
//    the same kernel family); where gemm_fp16 takes its 256x256 tile (large
//    prefill) exactly those two calls and swiglu, with the up projection in a
//    library buffer; and for shapes outside all of these (unaligned
//    operands, hidden % 64 != 0 at T > 4) swiglu_fused_direct: one thread per
//    output column and up to four tokens, fp32 fmaf over k in order -- the
//    arithmetic of the reference's naive kernel (src/kernels/gemm_fp16.cu:
//    241-262) for both projections.
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

// out[t, i] = swiglu(fp16(sum_k X[t,k] Wg[k,i]), fp16(sum_k X[t,k] Wu[k,i])),
// sums in fp32 with fmaf in k order; thread = column i, tokens t0..t0+TT-1.
// Weight reads are coalesced along i; X reads are the same address across
// the wave (one broadcast per k).
template <int TT>
__global__ void __launch_bounds__(256) swiglu_fused_direct(const uint16_t* X, const uint16_t* Wg,
                                                           const uint16_t* Wu, uint16_t* out, int T,
                                                           int H, int I) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * TT;
    if (i >= I) return;
    float g[TT], u[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) g[t] = u[t] = 0.0f;
    const uint16_t* xr[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) xr[t] = X + (int64_t)min(t0 + t, T - 1) * H;
    for (int k = 0; k < H; ++k) {
        const float wg = h2f(Wg[(int64_t)k * I + i]);
        const float wu = h2f(Wu[(int64_t)k * I + i]);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const float x = h2f(xr[t][k]);
            g[t] = fmaf(x, wg, g[t]);
            u[t] = fmaf(x, wu, u[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t)
        if (t0 + t < T) out[(int64_t)(t0 + t) * I + i] = swiglu_h(f2h(g[t]), f2h(u[t]));
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
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    // where gemm_fp16 takes the 256x256 tile for the projections (large
    // prefill), the same two calls and SwiGLU: gate into out, up into a
    // library buffer, SwiGLU in place -- the two-GEMM result by construction
    if (fp16_takes_big_tile(X, W_gate, out, T, inter, hidden, dev.num_cus) &&
        fp16_takes_big_tile(X, W_up, out, T, inter, hidden, dev.num_cus)) {
        void* ubuf = nullptr;
        if ((st = acquire_buffer(stream, kBufSwiglu, (size_t)T * inter * 2, &ubuf)) != CLOVE_OK) return st;
        uint16_t* up = static_cast<uint16_t*>(ubuf);
        if ((st = launch_gemm_fp16(X, W_gate, out, 1, T, inter, hidden, 1.0f, 0.0f, stream)) != CLOVE_OK) return st;
        if ((st = launch_gemm_fp16(X, W_up, up, 1, T, inter, hidden, 1.0f, 0.0f, stream)) != CLOVE_OK) return st;
        return launch_swiglu(out, up, out, (int64_t)T * inter, stream);
    }
    // (the kernel family gemm_fp16 takes for each projection: the skinny
    // kernel first where it would, then the GEMV for T <= 4)
    if (skinny_before_gemv(T, inter, hidden) &&
        try_skinny_swiglu(X, W_gate, W_up, out, T, hidden, inter, dev.num_cus, stream, &st))
        return st;
    if (try_gemv_swiglu(X, W_gate, W_up, out, T, hidden, inter, stream, &st)) return st;
    if (try_skinny_swiglu(X, W_gate, W_up, out, T, hidden, inter, dev.num_cus, stream, &st)) return st;
    constexpr int TT = 4;
    const dim3 grid((unsigned)hw::cdiv(inter, 256), (unsigned)hw::cdiv(T, TT));
    if (grid.y > 65535u) return CLOVE_ERR_INVALID_DIM;
    CLOVE_LAUNCH(act::swiglu_fused_direct<TT>, grid, dim3(256), 0, stream, X, W_gate, W_up, out, T, hidden,
                 inter);
    return check_launch();
}

}  // namespace clove
