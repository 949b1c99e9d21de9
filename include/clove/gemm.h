// C++ drop-in for the Clove Compute GEMM API on MI355X.
//
// Same namespace, function names, argument order and default arguments as the
// reference header include/clove/kernels/gemm.cuh:41-101, with hipStream_t in
// place of cudaStream_t.  Every call forwards to the C ABI in <clove/gemm_c.h>;
// a non-OK status is reported the reference's way (include/clove/common.cuh:11-21):
// print file:line and the error, then exit(EXIT_FAILURE).  <clove/common.h>
// brings the rest of the reference's common header: CLOVE_CHECK_CUDA /
// CLOVE_CHECK_LAST / CLOVE_SYNC_CHECK, cdiv, DType, dtype_size, CudaType.
#pragma once

#include <clove/common.h>
#include <clove/gemm_c.h>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace clove {

// include/clove/kernels/gemm.cuh:13-31: the FP16 GEMM's tile configuration,
// same member names.  The values describe this library's large-shape FP16
// kernel on gfx950: a 256x256x64 workgroup tile of four 64-wide waves, each
// wave a 128x128 tile of 16x16x32 fp16 MFMAs (fp32 accumulation).  Nothing in
// the library reads these; they are informational, as in the reference.
struct GemmConfig {
    static constexpr int BM = 256;  // workgroup tile M
    static constexpr int BN = 256;  // workgroup tile N
    static constexpr int BK = 64;   // workgroup tile K (one LDS stage)

    static constexpr int WM = 128;  // wave tile M
    static constexpr int WN = 128;  // wave tile N

    static constexpr int TM = 8;    // MFMA tiles per wave along M (WM / WMMA_M)
    static constexpr int TN = 8;    // MFMA tiles per wave along N (WN / WMMA_N)

    static constexpr int NUM_THREADS = 256;  // 4 waves of 64 lanes

    // matrix-core instruction shape (v_mfma_f32_16x16x32_f16); the reference
    // names it after WMMA
    static constexpr int WMMA_M = 16;
    static constexpr int WMMA_N = 16;
    static constexpr int WMMA_K = 32;
};

// include/clove/kernels/gemm.cuh:72
constexpr int INT4_GROUP_SIZE = CLOVE_INT4_GROUP_SIZE;

namespace detail {
inline void check(clove_status_t status, const char* file, int line) {
    if (status != CLOVE_OK) {
        std::fprintf(stderr, "clove error at %s:%d: %s\n", file, line,
                     clove_status_string(status));
        std::exit(EXIT_FAILURE);
    }
}
}  // namespace detail

#define CLOVE_CHECK_STATUS(call) ::clove::detail::check((call), __FILE__, __LINE__)

// include/clove/kernels/gemm.cuh:41-49
inline void gemm_fp16(const half* A, const half* B, half* C, int M, int N, int K,
                      float alpha = 1.0f, float beta = 0.0f, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_fp16(A, B, C, M, N, K, alpha, beta, stream));
}

// include/clove/kernels/gemm.cuh:57-65
inline void gemm_int8(const int8_t* A_q, const int8_t* B_q, half* C, int M, int N, int K,
                      float A_scale, int8_t A_zero, float B_scale, int8_t B_zero,
                      hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_int8(A_q, B_q, C, M, N, K, A_scale, A_zero, B_scale,
                                       B_zero, stream));
}

// include/clove/kernels/gemm.cuh:77-87
inline void gemm_int4(const uint8_t* A_q, const half* A_scale, const half* A_zero,
                      const uint8_t* B_q, const half* B_scale, const half* B_zero, half* C,
                      int M, int N, int K, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_int4(A_q, A_scale, A_zero, B_q, B_scale, B_zero, C, M, N,
                                       K, stream));
}

// include/clove/kernels/gemm.cuh:93-101
inline void gemm_fp16_batched(const half* A, const half* B, half* C, int batch, int M, int N,
                              int K, float alpha = 1.0f, float beta = 0.0f,
                              hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(
        clove_gemm_fp16_batched(A, B, C, batch, M, N, K, alpha, beta, stream));
}

// include/clove/kernels/activations.cuh:25-31
inline void swiglu(const half* gate, const half* up, half* output, int size,
                   hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_swiglu(gate, up, output, size, stream));
}

// include/clove/kernels/activations.cuh:37-46 (declared, never defined, in the
// reference)
inline void swiglu_fused(const half* input, const half* W_gate, const half* W_up, half* output,
                         int batch_seq, int hidden_dim, int intermediate_dim,
                         hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_swiglu_fused(input, W_gate, W_up, output, batch_seq, hidden_dim,
                                          intermediate_dim, stream));
}

// Extensions (no reference counterpart; see <clove/gemm_c.h>).
inline void gemm_int8_rowcol(const int8_t* A_q, const int8_t* B_q, const half* A_scale,
                             const half* B_scale, half* C, int M, int N, int K,
                             int8_t A_zero = 0, int8_t B_zero = 0, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_int8_rowcol(A_q, B_q, A_scale, B_scale, C, M, N, K, A_zero,
                                              B_zero, stream));
}

inline void gemm_int8_ex(const int8_t* A_q, const int8_t* B_q, half* C, int M, int N, int K,
                         float A_scale, int8_t A_zero, float B_scale, int8_t B_zero,
                         clove_int8_mode_t mode, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_int8_ex(A_q, B_q, C, M, N, K, A_scale, A_zero, B_scale,
                                          B_zero, (int)mode, stream));
}

inline void gemm_int4_ex(const uint8_t* A_q, const half* A_scale, const half* A_zero,
                         const uint8_t* B_q, const half* B_scale, const half* B_zero, half* C,
                         int M, int N, int K, clove_int4_mode_t mode, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_gemm_int4_ex(A_q, A_scale, A_zero, B_q, B_scale, B_zero, C, M, N,
                                          K, mode, stream));
}

inline void gemm_w4a16(const half* X, const uint8_t* W_q, const half* W_scale,
                       const half* W_zero, half* Y, int T, int O, int K, float alpha = 1.0f,
                       float beta = 0.0f, hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(
        clove_gemm_w4a16(X, W_q, W_scale, W_zero, Y, T, O, K, alpha, beta, stream));
}

inline void w4a16_swiglu(const half* X, const uint8_t* W_q, const half* W_scale,
                         const half* W_zero, half* H, int T, int I, int K,
                         hipStream_t stream = 0) {
    CLOVE_CHECK_STATUS(clove_w4a16_swiglu(X, W_q, W_scale, W_zero, H, T, I, K, stream));
}

}  // namespace clove
