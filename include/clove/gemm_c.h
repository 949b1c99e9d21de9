/*
 * clove_gemm C ABI -- MI355X (gfx950) GEMM hot path of Clove Compute.
 *
 * Plain C: raw device pointers, int dimensions, a status code.  Every entry
 * point is asynchronous on `stream` (a hipStream_t; NULL = the default stream),
 * does not synchronise the host, and validates its arguments before touching
 * the GPU.  Half-precision buffers are IEEE binary16 (passed as void*).
 * All matrices are dense row-major.  Output buffers must not overlap inputs.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the Clove Compute source tree).  The C++ spellings with the reference's
 * names, argument order and defaults live in <clove/gemm.h>.
 *
 * Scratch: split-K launches keep a per-(device, stream) scratch buffer that
 * the library allocates on first use (hipMalloc) and keeps until
 * clove_release_scratch() or process exit.  Calls on different streams never
 * share scratch; calls on one stream are ordered by the stream.  A call that
 * needs more scratch than the stream holds allocates a larger buffer (twice
 * the size or more) and keeps the old one until clove_release_scratch(), so
 * that calls of other host threads on the same stream that already took it
 * stay valid; no call synchronises a stream.
 */
#ifndef CLOVE_GEMM_C_H
#define CLOVE_GEMM_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum clove_status {
    CLOVE_OK = 0,
    CLOVE_ERR_NULL_POINTER = 1,   /* a required pointer is NULL */
    CLOVE_ERR_INVALID_DIM = 2,    /* a dimension is negative */
    CLOVE_ERR_INVALID_ARG = 3,    /* odd K for INT4, bad mode, misaligned half pointer */
    CLOVE_ERR_ALIASING = 4,       /* the output overlaps an input */
    CLOVE_ERR_OUT_OF_MEMORY = 5,  /* scratch allocation failed */
    CLOVE_ERR_LAUNCH = 6,         /* the HIP runtime rejected a launch */
    CLOVE_ERR_NO_DEVICE = 7,      /* no usable HIP device */
    CLOVE_ERR_WORKSPACE = 8,      /* the bound workspace is too small for the call */
    CLOVE_ERR_SCRATCH_LIMIT = 9   /* clove_gemm_fp16_noalloc: the call needs more scratch
                                     than CLOVE_NOALLOC_SCRATCH_BYTES */
} clove_status_t;

/* INT4 arithmetic selected by clove_gemm_int4_ex. */
typedef enum clove_int4_mode {
    /* per-128-group (q - zero) * scale on both operands, int32 partials per group
     * (the layout and scales the reference API declares) */
    CLOVE_INT4_GROUPWISE = 0,
    /* the reference kernel's arithmetic: q - 8, zeros ignored, whole-K integer
     * sum scaled by the last group's scales, B stride floor(N/2)
     * (src/kernels/gemm_int4.cu:45-193) */
    CLOVE_INT4_REFERENCE_LITERAL = 1
} clove_int4_mode_t;

/* include/clove/kernels/gemm.cuh:72 (INT4_GROUP_SIZE) */
#define CLOVE_INT4_GROUP_SIZE 128

/* Human-readable name of a status code (static storage). */
const char* clove_status_string(clove_status_t status);

/* ABI revision of this header; bumped on any signature change. */
int clove_abi_version(void);

/*
 * C = alpha * A @ B + beta * C.  A [M,K], B [K,N], C [M,N], fp16; fp32
 * accumulation and fp32 epilogue, fp16 round-to-nearest-even output.
 * beta == 0 never reads C.  M == 0 or N == 0 is a no-op; K == 0 gives beta*C.
 * Replaces clove::gemm_fp16 (include/clove/kernels/gemm.cuh:41-49,
 * src/kernels/gemm_fp16.cu:277-305).
 */
clove_status_t clove_gemm_fp16(const void* A, const void* B, void* C,
                               int M, int N, int K, float alpha, float beta,
                               void* stream);

/*
 * Batched clove_gemm_fp16 with contiguous batches: A [batch,M,K],
 * B [batch,K,N], C [batch,M,N].
 * Replaces clove::gemm_fp16_batched (include/clove/kernels/gemm.cuh:93-101,
 * src/kernels/gemm_fp16.cu:366-383).
 */
clove_status_t clove_gemm_fp16_batched(const void* A, const void* B, void* C,
                                       int batch, int M, int N, int K,
                                       float alpha, float beta, void* stream);

/*
 * W8A8 with per-tensor scale and zero point:
 *   acc = sum_k (A_q[m,k] - A_zero) * (B_q[k,n] - B_zero)      (int32, exact)
 *   C   = fp16( float(acc) * (A_scale * B_scale) )
 * A_q [M,K], B_q [K,N] int8; C [M,N] fp16.
 * Replaces clove::gemm_int8 (include/clove/kernels/gemm.cuh:57-65,
 * src/kernels/gemm_int8.cu:119-137).
 */
clove_status_t clove_gemm_int8(const int8_t* A_q, const int8_t* B_q, void* C,
                               int M, int N, int K,
                               float A_scale, int8_t A_zero,
                               float B_scale, int8_t B_zero, void* stream);

/* INT8 arithmetic modes of clove_gemm_int8_ex */
typedef enum {
    /* acc = sum over k < K only (clove_gemm_int8) */
    CLOVE_INT8_EXACT = 0,
    /* the reference kernel's accumulator at any K: it walks K in 32-wide tiles,
     * loads 0 for k >= K and subtracts the zero points from those zeros too, so
     * acc = exact + (32*ceil(K/32) - K) * A_zero * B_zero
     * (src/kernels/gemm_int8.cu:43, 52-54, 63-64, 89-93); equal to
     * CLOVE_INT8_EXACT when K % 32 == 0 or a zero point is 0 */
    CLOVE_INT8_REFERENCE_LITERAL = 1
} clove_int8_mode_t;

/*
 * clove_gemm_int8 with a choice of arithmetic mode (clove_int8_mode_t).
 * Extension of clove::gemm_int8 (include/clove/kernels/gemm.cuh:57-65).
 */
clove_status_t clove_gemm_int8_ex(const int8_t* A_q, const int8_t* B_q, void* C,
                                  int M, int N, int K,
                                  float A_scale, int8_t A_zero,
                                  float B_scale, int8_t B_zero, int mode, void* stream);

/*
 * W8A8 with fp16 per-row scales A_scale [M] (tokens) and per-column scales
 * B_scale [N] (output channels): C = fp16(float(acc) * (A_scale[m]*B_scale[n])).
 * With broadcast scales it equals clove_gemm_int8 bit for bit.  Extension of
 * clove::gemm_int8 (include/clove/kernels/gemm.cuh:57-65), which is per-tensor.
 */
clove_status_t clove_gemm_int8_rowcol(const int8_t* A_q, const int8_t* B_q,
                                      const void* A_scale, const void* B_scale,
                                      void* C, int M, int N, int K,
                                      int8_t A_zero, int8_t B_zero, void* stream);

/*
 * Test hook: the raw int32 accumulators [M,N] of the INT8 kernels (same kernels,
 * integer epilogue).  No reference counterpart: it exposes the bit-exact
 * accumulator the reference's gemm_int8_kernel keeps in registers
 * (src/kernels/gemm_int8.cu:37, :87-96).
 */
clove_status_t clove_gemm_int8_acc32(const int8_t* A_q, const int8_t* B_q,
                                     int32_t* acc, int M, int N, int K,
                                     int8_t A_zero, int8_t B_zero, void* stream);

/*
 * Packed INT4 x INT4 GEMM, group-wise (CLOVE_INT4_GROUPWISE):
 *   A_q [M, K/2]        two nibbles per byte, even k in the high nibble
 *   A_scale, A_zero     [M, ceil(K/128)] fp16
 *   B_q [K, ceil(N/2)]  two nibbles per byte along N, even n in the high nibble
 *   B_scale, B_zero     [ceil(K/128), N] fp16
 *   C [M,N] fp16 = sum_g A_scale[m,g]*B_scale[g,n] *
 *                  sum_{k in g} (qA - zA[m,g]) * (qB - zB[g,n])
 * Zero points are integer offsets stored as fp16 (non-integers round to nearest
 * even).  K must be even.  For even N the byte layout is the reference's.
 * Replaces clove::gemm_int4 (include/clove/kernels/gemm.cuh:77-87,
 * src/kernels/gemm_int4.cu:195-216).
 */
clove_status_t clove_gemm_int4(const uint8_t* A_q, const void* A_scale,
                               const void* A_zero, const uint8_t* B_q,
                               const void* B_scale, const void* B_zero, void* C,
                               int M, int N, int K, void* stream);

/*
 * Test hook: the per-group int32 partial sums of the group-wise INT4 GEMM,
 *   P[(m * N + n) * G + g] = sum_{k in group g} (qA[m,k] - zA[m,g]) * (qB[k,n] - zB[g,n])
 * (G = K / 128), the exact integers the int8-MFMA kernel folds into its fp32
 * accumulators (same pre-pass, same kernel, no fold), so that they can be
 * checked bit for bit.  No reference counterpart: the reference's
 * gemm_int4_kernel never forms per-group partials (src/kernels/gemm_int4.cu:
 * 137-190 sums every k before scaling).  Operands as clove_gemm_int4 (no
 * scales).  Domain: K a multiple of 256, A_q 16-byte aligned, P 4-byte aligned
 * (else CLOVE_ERR_INVALID_ARG); a partial whose row or column zero point lies
 * outside [-112, 127] is INT32_MIN.
 */
clove_status_t clove_gemm_int4_group_acc32(const uint8_t* A_q, const void* A_zero,
                                           const uint8_t* B_q, const void* B_zero,
                                           int32_t* P, int M, int N, int K, void* stream);

/* clove_gemm_int4 with an explicit arithmetic mode (see clove_int4_mode_t).
 * In CLOVE_INT4_REFERENCE_LITERAL mode B_q is [K, floor(N/2)] as in the
 * reference and the zero pointers may be NULL (never read). */
clove_status_t clove_gemm_int4_ex(const uint8_t* A_q, const void* A_scale,
                                  const void* A_zero, const uint8_t* B_q,
                                  const void* B_scale, const void* B_zero,
                                  void* C, int M, int N, int K,
                                  clove_int4_mode_t mode, void* stream);

/*
 * W4A16 linear layer: fp16 activations x group-128 INT4 weights.
 *   Y[t,o] = alpha * sum_k X[t,k] * (qW(o,k) - W_zero[o,g]) * W_scale[o,g]
 *            + beta * Y[t,o]
 * X [T,K] fp16, W_q [O, K/2] (gemm_int4's A layout), W_scale/W_zero [O, K/128]
 * fp16, Y [T,O] fp16.  beta = 1 is the residual add of the reference's o_proj
 * and down_proj (src/runtime/inference.cu:165-168, :191-194).  K even.
 * No reference entry point takes fp16 activations with INT4 weights; this is
 * the linear-layer call (src/runtime/inference.cu:139-194) on INT4 weights.
 */
clove_status_t clove_gemm_w4a16(const void* X, const uint8_t* W_q,
                                const void* W_scale, const void* W_zero, void* Y,
                                int T, int O, int K, float alpha, float beta,
                                void* stream);

/*
 * SwiGLU: output[i] = fp16(silu(gate[i]) * up[i]), silu(x) = x / (1 + exp(-x))
 * in fp32.  Replaces clove::swiglu (include/clove/kernels/activations.cuh:25-31,
 * src/kernels/activations.cu:76-134).  `output` may be `gate` or `up` (in place).
 */
clove_status_t clove_swiglu(const void* gate, const void* up, void* output, int size,
                            void* stream);

/*
 * Fused gate/up projections and SwiGLU on FP16 weights:
 *   output[t,i] = swiglu(fp16(input @ W_gate)[t,i], fp16(input @ W_up)[t,i])
 * input [batch_seq, hidden_dim], W_gate / W_up [hidden_dim, intermediate_dim]
 * (gemm_fp16's B layout), output [batch_seq, intermediate_dim], all fp16.
 * Replaces clove::swiglu_fused, declared in include/clove/kernels/
 * activations.cuh:37-46 and never defined there.  Where gemm_fp16 would run
 * each projection on its GEMV or skinny MFMA kernel (aligned operands, the
 * decode and small-batch shapes), one launch that writes neither projection
 * to memory: each output tile's gate and up sums are formed side by side in
 * the k order of those kernels, so the result equals gemm_fp16 x 2 followed
 * by clove_swiglu bit for bit, and the epilogue applies SwiGLU to their fp16
 * values.  Where gemm_fp16 takes its 256x256 tile (large prefill), exactly
 * those two calls and clove_swiglu, the up projection in a library buffer of
 * batch_seq x intermediate_dim fp16 (bit-identical by construction).  Other
 * shapes (unaligned operands, or hidden_dim % 64 != 0 beyond 4 rows): one
 * direct kernel with the reference naive kernel's fp32 k-order arithmetic for
 * both projections, within the FP16 tolerance of the two-call result.
 */
clove_status_t clove_swiglu_fused(const void* input, const void* W_gate, const void* W_up,
                                  void* output, int batch_seq, int hidden_dim,
                                  int intermediate_dim, void* stream);

/*
 * Fused MLP gate/up projections and SwiGLU on group-128 INT4 weights:
 *   H[t,i] = swiglu(gate[t,i], up[t,i]),
 *   gate = fp16(X @ dequant(W[0:I])^T),  up = fp16(X @ dequant(W[I:2I])^T)
 * X [T,K] fp16; W_q [2I, K/2] in gemm_int4's A layout with the I gate rows
 * first and the I up rows after them; W_scale / W_zero [2I, K/128] fp16;
 * H [T,I] fp16.  K even.  The reference MLP's gate and up gemm_fp16 calls and
 * its swiglu (src/runtime/inference.cu:172-186) in one pass that writes
 * neither projection to memory (when K % 128 == 0 and X, W_q are 16-byte
 * aligned, or T <= 4; other shapes run the two W4A16 layers and SwiGLU).
 */
clove_status_t clove_w4a16_swiglu(const void* X, const uint8_t* W_q, const void* W_scale,
                                  const void* W_zero, void* H, int T, int I, int K,
                                  void* stream);

/* Caller-owned workspace (no reference counterpart: the reference allocates no
 * scratch).  Per host thread, three modes:
 *
 *  - library scratch (the default): the per-(device, stream) buffers above;
 *  - a bound workspace, clove_workspace_bind(ptr, bytes): calls on this thread
 *    take their split-K partials, completion counters and intermediates from
 *    [ptr, ptr + bytes) and allocate nothing; a call that needs more returns
 *    CLOVE_ERR_WORKSPACE and launches nothing.  (No kernel uses private
 *    scratch either, which the library build checks.)  ptr must be 256-byte aligned
 *    and bytes >= CLOVE_WORKSPACE_MIN_BYTES; the first CLOVE_WORKSPACE_MIN_BYTES
 *    (the counters) must be zero before the first call, and every call leaves
 *    them zero.  Calls that may run at the same time on the device (other
 *    streams, other threads) must not share a workspace.
 *    clove_workspace_bind(NULL, 0) returns to library scratch;
 *  - a size query: between clove_workspace_query_begin() and
 *    clove_workspace_query_end(), calls on this thread validate their
 *    arguments and plan their launches but launch nothing and allocate
 *    nothing; query_end returns the largest workspace any of them needs
 *    (0 if none needs one) and restores the previous mode.  A query plans
 *    with the pointers it is given (alignment selects kernels), so pass the
 *    ones the real call will use. */
#define CLOVE_WORKSPACE_MIN_BYTES ((size_t)65536)
clove_status_t clove_workspace_bind(void* ptr, size_t bytes);
clove_status_t clove_workspace_query_begin(void);
size_t clove_workspace_query_end(void);

/*
 * clove_gemm_fp16 for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No reference counterpart.  Same arguments, kernels, split plans and results
 * (bit for bit) as clove_gemm_fp16; it calls no hipMalloc / hipFree and no
 * allocating library routine.  Its split-K partials and completion counters
 * live in a fixed device array of CLOVE_NOALLOC_SCRATCH_BYTES per GPU (the
 * library's static device memory, held until the process ends); a call that
 * would need more returns CLOVE_ERR_SCRATCH_LIMIT and launches nothing.
 * Every shape with M <= 512 and N, K <= 8192 whose operands are 16-byte
 * aligned, with N % 8 == 0 and K % 64 == 0, fits, as does every shape on the
 * 256x256 tile (its K split needs at most 64 MiB of partials).  The first call on a device clears the array's counters
 * with one small kernel on `stream`.  Every call on a GPU shares that GPU's
 * array: calls that may overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Inside a workspace
 * size query it validates and plans as clove_gemm_fp16, returns
 * CLOVE_ERR_SCRATCH_LIMIT for a call the array cannot hold, and leaves the
 * query's size as it was (the array is not the caller's workspace).
 */
#define CLOVE_NOALLOC_SCRATCH_BYTES ((size_t)65 << 20)
clove_status_t clove_gemm_fp16_noalloc(const void* A, const void* B, void* C,
                                       int M, int N, int K, float alpha, float beta,
                                       void* stream);

/* Frees the scratch buffers held for the current device (all streams),
 * including the SwiGLU intermediates and buffers replaced by larger ones.
 * Synchronises the device first; no other call may be using the library on
 * this device meanwhile.  No reference counterpart. */
clove_status_t clove_release_scratch(void);

#ifdef __cplusplus
}
#endif

#endif /* CLOVE_GEMM_C_H */
