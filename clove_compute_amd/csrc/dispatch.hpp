// Internal interface between the C ABI layer (capi.hip) and the kernel
// launchers (gemm_*.hip).  Not installed; no reference counterpart.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "clove/gemm_c.h"

namespace clove {

// Per-(device, stream) scratch for split-K partials and completion counters.
// Counters are zero between launches (each last-arriving workgroup resets its
// own counter), so a launch may use them without clearing.
struct Scratch {
    float* partials = nullptr;
    size_t partial_bytes = 0;
    unsigned* counters = nullptr;
    size_t num_counters = 0;
};

// Returns scratch with at least the requested capacity for `stream` on the
// current device (implemented in capi.hip): library-owned, or carved from the
// workspace the calling thread has bound (clove_workspace_bind), or, in a
// workspace size query, a placeholder that only records the size.
clove_status_t acquire_scratch(hipStream_t stream, size_t partial_bytes, size_t num_counters,
                               Scratch* out);

// True while the calling thread runs a workspace size query: calls plan and
// size their scratch but launch nothing.
bool dry_run();

// Every kernel launch of the library goes through this.
#define CLOVE_LAUNCH(...)                                   \
    do {                                                    \
        if (!::clove::dry_run()) hipLaunchKernelGGL(__VA_ARGS__); \
    } while (0)

struct DeviceInfo {
    int device = 0;
    int num_cus = 256;
};
clove_status_t current_device_info(DeviceInfo* out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

clove_status_t launch_gemm_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C, int batch,
                                int M, int N, int K, float alpha, float beta,
                                hipStream_t stream);

enum class Int8Out { kHalfPerTensor, kHalfRowCol, kAcc32 };

struct Int8Args {
    const int8_t* A = nullptr;
    const int8_t* B = nullptr;
    void* C = nullptr;  // uint16_t* (fp16) or int32_t* (kAcc32)
    const uint16_t* sa = nullptr;  // [M] fp16 (kHalfRowCol)
    const uint16_t* sb = nullptr;  // [N] fp16 (kHalfRowCol)
    float scale = 1.0f;            // A_scale * B_scale (kHalfPerTensor)
    int za = 0, zb = 0;
    // added to every int32 accumulator (wrap-around): (32 ceil(K/32) - K) za zb
    // in the reference-literal mode, else 0; only the kernels that take zero
    // points apply it (it is 0 whenever a zero point is)
    int acc_add = 0;
    int M = 0, N = 0, K = 0;
    Int8Out out = Int8Out::kHalfPerTensor;
};
clove_status_t launch_gemm_int8(const Int8Args& args, hipStream_t stream);

struct Int4Args {
    const uint8_t* A = nullptr;
    const uint16_t* A_scale = nullptr;
    const uint16_t* A_zero = nullptr;
    const uint8_t* B = nullptr;
    const uint16_t* B_scale = nullptr;
    const uint16_t* B_zero = nullptr;
    uint16_t* C = nullptr;
    int M = 0, N = 0, K = 0;
    clove_int4_mode_t mode = CLOVE_INT4_GROUPWISE;
};
clove_status_t launch_gemm_int4(const Int4Args& args, hipStream_t stream);

struct W4A16Args {
    const uint16_t* X = nullptr;
    const uint8_t* W = nullptr;
    const uint16_t* scale = nullptr;
    const uint16_t* zero = nullptr;
    uint16_t* Y = nullptr;
    int T = 0, O = 0, K = 0;
    float alpha = 1.0f, beta = 0.0f;
};
clove_status_t launch_w4a16(const W4A16Args& args, hipStream_t stream);

// MFMA path for INT4 weight rows x fp16 activations (i4w_gemm.hip).  Each
// returns false, launching nothing, when the shape or alignment is outside
// what the kernel handles (the caller then takes its general path); otherwise
// it launches and stores the launch status in *status.
bool try_i4w_w4a16(const W4A16Args& args, int num_cus, hipStream_t stream, clove_status_t* status);
bool try_i4w_int4(const Int4Args& args, int num_cus, hipStream_t stream, clove_status_t* status);
// group-wise INT4 x INT4 on int8 MFMA (i4i4_gemm.hip): N >= 64, K % 256 == 0,
// 16-byte aligned A; zero points in [-112, 127] (others give NaN outputs)
bool try_i4i4(const Int4Args& args, int num_cus, hipStream_t stream, clove_status_t* status);
// the int8-MFMA kernel's per-group int32 sums P [M, N, G] (test hook; group-wise)
clove_status_t launch_i4i4_partials(const Int4Args& args, int32_t* P, int num_cus, hipStream_t stream);
// SwiGLU of a fused gate/up INT4 weight: args.W holds 2 args.O rows (gate rows,
// then up rows, scales / zeros likewise), args.Y receives H [T, O]
bool try_i4w_w4a16_swiglu(const W4A16Args& args, int num_cus, hipStream_t stream, clove_status_t* status);

// H [T, O] = swiglu(X @ gate^T, X @ up^T) on a fused gate/up W4A16 weight
// (w4a16.hip): GEMV for T <= 4, the INT4-weight MFMA GEMM above, or, for shapes
// neither covers, the two linear layers and the elementwise SwiGLU
clove_status_t launch_w4a16_swiglu(const W4A16Args& args, hipStream_t stream);
// out[i] = swiglu(gate[i], up[i]), n elements (swiglu.hip)
clove_status_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                             hipStream_t stream);
// out [T, inter] = swiglu(X @ W_gate, X @ W_up), FP16 weights [hidden, inter]
clove_status_t launch_swiglu_fused_fp16(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up,
                                        uint16_t* out, int T, int hidden, int inter, hipStream_t stream);

// A device buffer of at least `bytes` owned by the library per (device,
// stream, slot), kept across calls (capi.hip), or carved from the bound
// workspace as acquire_scratch; slot 0 is reserved for the split-K scratch.
clove_status_t acquire_buffer(hipStream_t stream, int slot, size_t bytes, void** out);
constexpr int kBufSwiglu = 1;  // gate / up intermediates of the unfused SwiGLU paths

// FP16 with two to four rows of A: the skinny MFMA kernel rather than the
// GEMV once the weight is large (cold, measured: 11008 x 4096 at M = 2 / 3 /
// 4: 21.1 / 21.3 / 21.0 us against 26.5 / 32.2 / 31.8 on the GEMV; 4096 x 4096
// at M = 3: 12.6 against 13.8; 2048 x 2048 at M = 3 and 4096 x 4096 at M = 2
// stay on the GEMV: 9.6 against 12.6, 11.8 against 12.6).  gemm_fp16 and the
// fused SwiGLU take the same decision per projection.
inline bool skinny_before_gemv(int M, int N, int K) {
    const int64_t nk = (int64_t)N * K;
    return M >= 2 && M <= 4 && nk > (M == 2 ? ((int64_t)24 << 20) : ((int64_t)5 << 20));
}

// MFMA path for few rows of A against a large N-contiguous B (skinny_gemm.hip):
// FP16 (any alpha/beta, batched) and INT8 with zero points 0.  Same contract
// as the try_i4w_* functions.
bool try_skinny_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C, int batch, int M, int N, int K,
                     float alpha, float beta, int num_cus, hipStream_t stream, clove_status_t* status);
bool try_skinny_int8(const Int8Args& args, int num_cus, hipStream_t stream, clove_status_t* status);
// out [T, inter] = swiglu(fp16(X @ W_gate), fp16(X @ W_up)) in one pass of the
// skinny kernel with two B operands (T > 4, or skinny_before_gemv; aligned,
// hidden % 64 == 0); same
// tiles and split plan as try_skinny_fp16 picks for each projection
bool try_skinny_swiglu(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up, uint16_t* out, int T,
                       int hidden, int inter, int num_cus, hipStream_t stream, clove_status_t* status);
// the same for T <= 4 on the FP16 GEMV (gemm_fp16.hip): each workgroup streams
// 128 columns of W_gate and the same 128 columns of W_up; false when the
// operands are not 16-byte aligned or hidden / inter are not multiples of 8
// true when launch_gemm_fp16 runs one (unbatched) M x N x K product on the
// 256x256 LDS-DMA tile (dma::gemm_f16_big)
bool fp16_takes_big_tile(const void* A, const void* B, const void* C, int M, int N, int K, int cus);
bool try_gemv_swiglu(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up, uint16_t* out, int T,
                     int hidden, int inter, hipStream_t stream, clove_status_t* status);

inline clove_status_t check_launch() {
    return hipGetLastError() == hipSuccess ? CLOVE_OK : CLOVE_ERR_LAUNCH;
}

// Raises a kernel's dynamic-LDS limit to `bytes` (needed above 64 KB) once per
// (device, kernel): the setting is per device and lasts for the process, so
// later calls only look it up.
clove_status_t ensure_lds(const void* kernel, int bytes);

}  // namespace clove
