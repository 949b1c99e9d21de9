/*
 * CPU oracle for the Clove Compute GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP kernels
 * are compared against, and the CPU baseline that bench.py times beside them.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library (clove_compute_amd/) never links, loads or calls it.
 *
 * Every function restates the per-element arithmetic of one reference routine
 * and cites the reference file:line it follows.  Half-precision values travel
 * as raw IEEE binary16 bit patterns (uint16_t), so no compiler half type is
 * involved.  Dimensions are int like the reference API; internal offsets are
 * 64-bit.
 *
 * How each function is pinned (the checks live in tests/test_oracle.py):
 *   f16 conversions     exhaustive against numpy's IEEE conversions
 *   gemm_fp16           numpy float64 matmul within a forward-error bound; bit
 *                       exact on small-integer inputs, identity B, K=1, alpha/beta
 *                       closed forms; committed golden vectors
 *   gemm_fp16_batched   equals per-batch gemm_fp16 (strides) + same closed forms
 *   gemm_int8(_rowcol)  int32 accumulators equal numpy int64 matmul of the
 *                       zero-shifted operands; epilogue equals numpy float32
 *   gemm_int4_literal   numpy matmul of unpacked nibbles (q-8), last-group scales,
 *                       N=1 and odd-N zero columns
 *   gemm_int4_groupwise per-group int32 partials equal numpy int64 einsum; output
 *                       within tolerance of float64; bit exact on power-of-two
 *                       scale cases
 *   w4a16               numpy float64 dequantised matmul
 */
#ifndef CLOVE_ORACLE_H
#define CLOVE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round-to-nearest-even on the narrowing side. */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_f32_to_f16_array(const float* x, uint16_t* h, int64_t n);
void oracle_f16_to_f32_array(const uint16_t* h, float* x, int64_t n);

/* C = alpha * A @ B + beta * C, fp16 in/out, fp32 sequential-k FMA.
 * Rows [m0, m1) only (m0=0, m1=M for the whole product); the bench times a
 * bounded row sample through this entry.  A [M,K], B [K,N], C [M,N] row-major. */
void oracle_gemm_fp16_rows(const uint16_t* A, const uint16_t* B, uint16_t* C,
                           int M, int N, int K, float alpha, float beta,
                           int m0, int m1);
void oracle_gemm_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C,
                      int M, int N, int K, float alpha, float beta);
/* oracle_gemm_fp16_rows with the rows spread over `nthreads` POSIX threads
 * (bit-identical to it: every element is one thread's sequential-k sum).
 * Returns the number of threads started (the rest run on the caller), -1 if
 * out of memory.  Used by the bench's all-cores CPU baseline. */
int oracle_gemm_fp16_rows_mt(const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K, float alpha, float beta,
                             int m0, int m1, int nthreads);

/* Unrounded float64 value of alpha * A @ B + beta * C_in (C_in may be NULL). */
void oracle_gemm_fp16_f64(const uint16_t* A, const uint16_t* B,
                          const uint16_t* C_in, double* out,
                          int M, int N, int K, double alpha, double beta);

/* Batched: A [batch,M,K], B [batch,K,N], C [batch,M,N]. */
void oracle_gemm_fp16_batched(const uint16_t* A, const uint16_t* B, uint16_t* C,
                              int batch, int M, int N, int K,
                              float alpha, float beta);

/* W8A8, per-tensor scale and zero.  acc_out (nullable) receives the int32
 * accumulators [M,N]. */
void oracle_gemm_int8(const int8_t* A_q, const int8_t* B_q, uint16_t* C,
                      int32_t* acc_out, int M, int N, int K,
                      float A_scale, int8_t A_zero, float B_scale, int8_t B_zero);

/* W8A8 as the reference kernel computes it at any K: 32-wide K tiles whose
 * bytes past K load as 0 before the zero points are subtracted, so every padded
 * k adds A_zero * B_zero (gemm_int8.cu:43-96). */
void oracle_gemm_int8_literal(const int8_t* A_q, const int8_t* B_q, uint16_t* C,
                              int32_t* acc_out, int M, int N, int K,
                              float A_scale, int8_t A_zero, float B_scale, int8_t B_zero);

/* W8A8 with fp16 per-row scales sa [M] and per-column scales sb [N]. */
void oracle_gemm_int8_rowcol(const int8_t* A_q, const int8_t* B_q,
                             const uint16_t* sa, const uint16_t* sb, uint16_t* C,
                             int32_t* acc_out, int M, int N, int K,
                             int8_t A_zero, int8_t B_zero);

/* INT4, the reference's literal arithmetic: nibbles decoded as q-8, zeros
 * ignored, the whole-K integer sum scaled by the LAST group's scales.
 * B_q uses the reference's stride floor(N/2); columns n >= 2*floor(N/2) read
 * no B data and produce 0 * scales. */
void oracle_gemm_int4_literal(const uint8_t* A_q, const uint16_t* A_scale,
                              const uint8_t* B_q, const uint16_t* B_scale,
                              uint16_t* C, int M, int N, int K);

/* INT4, group-wise dequantisation (group 128 along K):
 *   P_g[m,n] = sum_{k in g} (qA - zA[m,g]) * (qB - zB[g,n])     (int32, exact)
 *   C[m,n]   = f16( sum_g fma(f32(sA[m,g]) * f32(sB[g,n]), f32(P_g), acc) )
 * Zero points are fp16 values rounded to the nearest integer (ties to even).
 * B_q is [K, ceil(N/2)], high nibble = even column.
 * partials (nullable) receives P_g as [M, N, G]; out64 (nullable) receives the
 * float64 value sum_g sA*sB*P_g before rounding. */
void oracle_gemm_int4_groupwise(const uint8_t* A_q, const uint16_t* A_scale,
                                const uint16_t* A_zero, const uint8_t* B_q,
                                const uint16_t* B_scale, const uint16_t* B_zero,
                                uint16_t* C, int32_t* partials, double* out64,
                                int M, int N, int K);

/* W4A16 linear: Y[t,o] = alpha * sum_k X[t,k] * (qW(o,k) - z[o,g]) * s[o,g]
 *                        + beta * Y_in[t,o]
 * X [T,K] fp16, W_q [O,K/2] (high nibble = even k), W_scale/W_zero [O,G].
 * out64 (nullable) receives the float64 value; Y (nullable) its fp16 rounding.
 * Y_in may be NULL when beta == 0. */
void oracle_w4a16(const uint16_t* X, const uint8_t* W_q, const uint16_t* W_scale,
                  const uint16_t* W_zero, const uint16_t* Y_in, uint16_t* Y,
                  double* out64, int T, int O, int K, double alpha, double beta);

/* out[i] = fp16(silu(f32(gate[i])) * f32(up[i])), silu(x) = x / (1 + expf(-x))
 * in fp32 (src/kernels/activations.cu:9-11, :76-134). */
void oracle_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* CLOVE_ORACLE_H */
