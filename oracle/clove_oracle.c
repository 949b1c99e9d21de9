/*
 * CPU oracle for the Clove Compute GEMM hot path -- TEST INFRASTRUCTURE ONLY.
 * See clove_oracle.h for the contract and for how each function is pinned.
 * Built by oracle/Makefile with gcc; never linked into the product library.
 */
#include "clove_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 128

/* ------------------------------------------------------------------------- */
/* IEEE binary16 conversions (written from the IEEE 754 encoding).           */
/* ------------------------------------------------------------------------- */

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {                 /* NaN: quiet, keep top payload bits */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) {                /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                 /* below 2^-14: binary16 subnormal */
        if (ax < 0x33000000u) return (uint16_t)sign;   /* < 2^-25 (tie at 2^-25 -> 0) */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;    /* value * 2^24 = m * 2^-(shift) */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    const uint32_t e = (ax >> 23) - 127u + 15u;
    const uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* carry may bump exponent */
    return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {                            /* subnormal: m * 2^-24, exact in fp32 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void oracle_f32_to_f16_array(const float* x, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = oracle_f32_to_f16(x[i]);
}

void oracle_f16_to_f32_array(const uint16_t* h, float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = oracle_f16_to_f32(h[i]);
}

static float* widen(const uint16_t* h, int64_t n) {
    float* f = (float*)malloc((size_t)n * sizeof(float));
    if (f) oracle_f16_to_f32_array(h, f, n);
    return f;
}

/* ------------------------------------------------------------------------- */
/* FP16 GEMM                                                                  */
/* ------------------------------------------------------------------------- */

/*
 * Restates gemm_fp16_naive_kernel (src/kernels/gemm_fp16.cu:223-271):
 *   sum = 0f; for k in 0..K-1: sum += f32(A[m,k]) * f32(B[k,n])   (:241-262)
 * (contracted to one fused multiply-add per k), then
 *   r = alpha * sum; if beta != 0: r += beta * f32(C[m,n]); C = f16(r)  (:264-270)
 * The loop runs i-k-j so that each output keeps its own sequential k order.
 */
void oracle_gemm_fp16_rows(const uint16_t* A, const uint16_t* B, uint16_t* C,
                           int M, int N, int K, float alpha, float beta,
                           int m0, int m1) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    if (m0 < 0) m0 = 0;
    if (m1 > M) m1 = M;
    float* Bf = widen(B, (int64_t)K * N);
    float* s = (float*)malloc((size_t)N * sizeof(float));
    if (!Bf || !s) { free(Bf); free(s); return; }
    for (int m = m0; m < m1; m++) {
        for (int n = 0; n < N; n++) s[n] = 0.0f;
        const uint16_t* Arow = A + (int64_t)m * K;
        for (int k = 0; k < K; k++) {
            const float a = oracle_f16_to_f32(Arow[k]);
            const float* Brow = Bf + (int64_t)k * N;
            for (int n = 0; n < N; n++) s[n] = fmaf(a, Brow[n], s[n]);
        }
        uint16_t* Crow = C + (int64_t)m * N;
        for (int n = 0; n < N; n++) {
            float r = alpha * s[n];
            if (beta != 0.0f) r = fmaf(beta, oracle_f16_to_f32(Crow[n]), r);
            Crow[n] = oracle_f32_to_f16(r);
        }
    }
    free(Bf);
    free(s);
}

void oracle_gemm_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C,
                      int M, int N, int K, float alpha, float beta) {
    oracle_gemm_fp16_rows(A, B, C, M, N, K, alpha, beta, 0, M);
}

/* The same arithmetic as oracle_gemm_fp16_rows (per-element sequential k,
 * fp32 fmaf, the same epilogue), rows [m0, m1) split over `nthreads` POSIX
 * threads: thread t takes rows m0 + t, m0 + t + nthreads, ...  B is widened
 * once and shared.  Each output element is computed by exactly one thread in
 * the single-thread order, so the result is bit-identical to
 * oracle_gemm_fp16_rows for any thread count. */
struct fp16_mt_job {
    const uint16_t* A;
    const float* Bf;
    uint16_t* C;
    int N, K, m0, m1, t, nt;
    float alpha, beta;
};

static void* fp16_mt_worker(void* arg) {
    const struct fp16_mt_job* j = (const struct fp16_mt_job*)arg;
    float* s = (float*)malloc((size_t)j->N * sizeof(float));
    if (!s) return NULL;
    for (int m = j->m0 + j->t; m < j->m1; m += j->nt) {
        for (int n = 0; n < j->N; n++) s[n] = 0.0f;
        const uint16_t* Arow = j->A + (int64_t)m * j->K;
        for (int k = 0; k < j->K; k++) {
            const float a = oracle_f16_to_f32(Arow[k]);
            const float* Brow = j->Bf + (int64_t)k * j->N;
            for (int n = 0; n < j->N; n++) s[n] = fmaf(a, Brow[n], s[n]);
        }
        uint16_t* Crow = j->C + (int64_t)m * j->N;
        for (int n = 0; n < j->N; n++) {
            float r = j->alpha * s[n];
            if (j->beta != 0.0f) r = fmaf(j->beta, oracle_f16_to_f32(Crow[n]), r);
            Crow[n] = oracle_f32_to_f16(r);
        }
    }
    free(s);
    return NULL;
}

int oracle_gemm_fp16_rows_mt(const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K, float alpha, float beta,
                             int m0, int m1, int nthreads) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (m0 < 0) m0 = 0;
    if (m1 > M) m1 = M;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    float* Bf = widen(B, (int64_t)K * N);
    if (!Bf) return -1;
    pthread_t th[256];
    struct fp16_mt_job jobs[256];
    int started = 0;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (struct fp16_mt_job){A, Bf, C, N, K, m0, m1, t, nthreads, alpha, beta};
        if (pthread_create(&th[t], NULL, fp16_mt_worker, &jobs[t]) != 0) break;
        started++;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    /* rows of threads that could not start: computed here, same order */
    for (int t = started; t < nthreads; t++) fp16_mt_worker(&jobs[t]);
    free(Bf);
    return started;
}

void oracle_gemm_fp16_f64(const uint16_t* A, const uint16_t* B,
                          const uint16_t* C_in, double* out,
                          int M, int N, int K, double alpha, double beta) {
    if (M <= 0 || N <= 0) return;
    float* Bf = widen(B, (int64_t)K * N);
    double* s = (double*)malloc((size_t)N * sizeof(double));
    if ((!Bf && K > 0) || !s) { free(Bf); free(s); return; }
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) s[n] = 0.0;
        for (int k = 0; k < K; k++) {
            const double a = (double)oracle_f16_to_f32(A[(int64_t)m * K + k]);
            const float* Brow = Bf + (int64_t)k * N;
            for (int n = 0; n < N; n++) s[n] += a * (double)Brow[n];
        }
        for (int n = 0; n < N; n++) {
            double r = alpha * s[n];
            if (C_in && beta != 0.0) r += beta * (double)oracle_f16_to_f32(C_in[(int64_t)m * N + n]);
            out[(int64_t)m * N + n] = r;
        }
    }
    free(Bf);
    free(s);
}

/* Restates gemm_fp16_batched_kernel (src/kernels/gemm_fp16.cu:311-364): the
 * naive arithmetic per batch at offsets b*M*K, b*K*N, b*M*N (:320-322). */
void oracle_gemm_fp16_batched(const uint16_t* A, const uint16_t* B, uint16_t* C,
                              int batch, int M, int N, int K,
                              float alpha, float beta) {
    for (int b = 0; b < batch; b++) {
        oracle_gemm_fp16(A + (int64_t)b * M * K, B + (int64_t)b * K * N,
                         C + (int64_t)b * M * N, M, N, K, alpha, beta);
    }
}

/* ------------------------------------------------------------------------- */
/* INT8 GEMM                                                                  */
/* ------------------------------------------------------------------------- */

/* int32 accumulators acc[m,n] = sum_k (a - za) * (b - zb), i-k-j order
 * (src/kernels/gemm_int8.cu:87-96).  Products and sums fit int32 at K <= 33025. */
static int32_t* int8_accumulate(const int8_t* A_q, const int8_t* B_q,
                                int M, int N, int K, int za, int zb) {
    int32_t* acc = (int32_t*)calloc((size_t)M * N, sizeof(int32_t));
    int32_t* bcol = (int32_t*)malloc((size_t)N * sizeof(int32_t));
    if (!acc || !bcol) { free(acc); free(bcol); return NULL; }
    for (int m = 0; m < M; m++) {
        int32_t* arow = acc + (int64_t)m * N;
        for (int k = 0; k < K; k++) {
            const int32_t a = (int32_t)A_q[(int64_t)m * K + k] - za;
            const int8_t* brow = B_q + (int64_t)k * N;
            for (int n = 0; n < N; n++) bcol[n] = (int32_t)brow[n] - zb;
            for (int n = 0; n < N; n++) arow[n] += a * bcol[n];
        }
    }
    free(bcol);
    return acc;
}

/* Restates gemm_int8_kernel (src/kernels/gemm_int8.cu:16-117) as intended per
 * element: combined = A_scale * B_scale (fp32, :40), C = f16(f32(acc) * combined)
 * (:113-114).  The reference's thread map writes outside its 64x64 tile; this is
 * the formula its owning block computes. */
void oracle_gemm_int8(const int8_t* A_q, const int8_t* B_q, uint16_t* C,
                      int32_t* acc_out, int M, int N, int K,
                      float A_scale, int8_t A_zero, float B_scale, int8_t B_zero) {
    if (M <= 0 || N <= 0) return;
    int32_t* acc = int8_accumulate(A_q, B_q, M, N, K, A_zero, B_zero);
    if (!acc) return;
    const float combined = A_scale * B_scale;
    for (int64_t i = 0; i < (int64_t)M * N; i++) {
        if (C) C[i] = oracle_f32_to_f16((float)acc[i] * combined);
        if (acc_out) acc_out[i] = acc[i];
    }
    free(acc);
}

/* The reference kernel's own arithmetic at any K, as its owning block runs it
 * (src/kernels/gemm_int8.cu:43-96): K is walked in 32-wide tiles (:43), bytes
 * at k >= K are loaded as 0 (:52-54, :63-64), and the zero points are
 * subtracted from every loaded byte (:89-93), so each of the 32*ceil(K/32) - K
 * padded k of the last tile adds (0 - A_zero) * (0 - B_zero).  Epilogue as
 * oracle_gemm_int8 (:40, :113-114). */
void oracle_gemm_int8_literal(const int8_t* A_q, const int8_t* B_q, uint16_t* C,
                              int32_t* acc_out, int M, int N, int K,
                              float A_scale, int8_t A_zero, float B_scale, int8_t B_zero) {
    if (M <= 0 || N <= 0) return;
    const int BK = 32;
    const float combined = A_scale * B_scale;
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            uint32_t acc = 0; /* int32 with wrap-around, like the reference's int */
            for (int k0 = 0; k0 < K; k0 += BK) {
                for (int kk = 0; kk < BK; kk++) {
                    const int k = k0 + kk;
                    const int a = k < K ? A_q[(int64_t)m * K + k] : 0;
                    const int b = k < K ? B_q[(int64_t)k * N + n] : 0;
                    acc += (uint32_t)((a - (int)A_zero) * (b - (int)B_zero));
                }
            }
            const int64_t i = (int64_t)m * N + n;
            if (C) C[i] = oracle_f32_to_f16((float)(int32_t)acc * combined);
            if (acc_out) acc_out[i] = (int32_t)acc;
        }
    }
}

/* Row/column-scale extension of the same formula: combined = sa[m] * sb[n]. */
void oracle_gemm_int8_rowcol(const int8_t* A_q, const int8_t* B_q,
                             const uint16_t* sa, const uint16_t* sb, uint16_t* C,
                             int32_t* acc_out, int M, int N, int K,
                             int8_t A_zero, int8_t B_zero) {
    if (M <= 0 || N <= 0) return;
    int32_t* acc = int8_accumulate(A_q, B_q, M, N, K, A_zero, B_zero);
    if (!acc) return;
    for (int m = 0; m < M; m++) {
        const float fa = oracle_f16_to_f32(sa[m]);
        for (int n = 0; n < N; n++) {
            const int64_t i = (int64_t)m * N + n;
            const float combined = fa * oracle_f16_to_f32(sb[n]);
            if (C) C[i] = oracle_f32_to_f16((float)acc[i] * combined);
            if (acc_out) acc_out[i] = acc[i];
        }
    }
    free(acc);
}

/* ------------------------------------------------------------------------- */
/* INT4 GEMM                                                                  */
/* ------------------------------------------------------------------------- */

/* Nibble k of a packed row: even k in the high nibble, odd k in the low nibble
 * (src/kernels/gemm_int4.cu:27-34, :88-92). */
static inline int nib(const uint8_t* row, int k) {
    const uint8_t b = row[k >> 1];
    return (k & 1) ? (b & 0x0f) : (b >> 4);
}

/*
 * Restates gemm_int4_kernel (src/kernels/gemm_int4.cu:45-193) literally:
 *  - A nibbles (q-8) from A_q[m*(K/2) + k/2]                 (:81-97)
 *  - B nibbles (q-8) from B_q[k*(N/2) + n/2], zero when n/2 >= N/2 (:101-117)
 *  - fp32 sum over all K (exact for integers)                (:137-156)
 *  - scales of group g* = ((ceil(K/64)-1)*64)/128, i.e. the last K tile's
 *    group, remain in shared memory after the loop            (:77, :119-131)
 *  - C = f16((acc * a_s) * b_s)                              (:185-190)
 *  - A_zero and B_zero are never read.
 */
void oracle_gemm_int4_literal(const uint8_t* A_q, const uint16_t* A_scale,
                              const uint8_t* B_q, const uint16_t* B_scale,
                              uint16_t* C, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    const int G = (K + GROUP - 1) / GROUP;
    const int g_last = (((K + 63) / 64 - 1) * 64) / GROUP;
    const int half_n = N / 2;
    const int half_k = K / 2;
    float* acc = (float*)malloc((size_t)N * sizeof(float));
    if (!acc) return;
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) acc[n] = 0.0f;
        const uint8_t* arow = A_q + (int64_t)m * half_k;
        for (int k = 0; k < 2 * half_k; k++) {
            const float a = (float)(nib(arow, k) - 8);
            const uint8_t* brow = B_q + (int64_t)k * half_n;
            for (int n = 0; n < N; n++) {
                float b = 0.0f;
                if ((n >> 1) < half_n) b = (float)(nib(brow, n) - 8);
                acc[n] += a * b;
            }
        }
        const float a_s = oracle_f16_to_f32(A_scale[(int64_t)m * G + g_last]);
        for (int n = 0; n < N; n++) {
            const float b_s = oracle_f16_to_f32(B_scale[(int64_t)g_last * N + n]);
            C[(int64_t)m * N + n] = oracle_f32_to_f16(acc[n] * a_s * b_s);
        }
    }
    free(acc);
}

/* fp16 zero point -> integer offset, nearest with ties to even. */
static inline int zero_int(uint16_t h) {
    return (int)nearbyintf(oracle_f16_to_f32(h));
}

/*
 * Group-wise dequantised INT4 GEMM: the semantics the reference's API describes
 * (include/clove/kernels/gemm.cuh:71-87: per-group scales/zeros [M, K/128] and
 * [K/128, N], group size INT4_GROUP_SIZE = 128) and that its kernel leaves
 * unfinished (src/kernels/gemm_int4.cu:170-171).  Nibble order follows :27-34.
 */
void oracle_gemm_int4_groupwise(const uint8_t* A_q, const uint16_t* A_scale,
                                const uint16_t* A_zero, const uint8_t* B_q,
                                const uint16_t* B_scale, const uint16_t* B_zero,
                                uint16_t* C, int32_t* partials, double* out64,
                                int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    const int G = (K + GROUP - 1) / GROUP;
    const int bstride = (N + 1) / 2;
    const int half_k = K / 2;
    int32_t* vb = (int32_t*)malloc((size_t)K * N * sizeof(int32_t));
    int32_t* P = (int32_t*)malloc((size_t)N * sizeof(int32_t));
    if (!vb || !P) { free(vb); free(P); return; }
    /* unpacked, zero-shifted B: vb[k*N + n] = qB - zB[g,n] */
    for (int k = 0; k < K; k++) {
        const int g = k / GROUP;
        for (int n = 0; n < N; n++) {
            vb[(int64_t)k * N + n] = nib(B_q + (int64_t)k * bstride, n) -
                                     zero_int(B_zero[(int64_t)g * N + n]);
        }
    }
    for (int m = 0; m < M; m++) {
        const uint8_t* arow = A_q + (int64_t)m * half_k;
        float* accf = NULL;
        double* accd = NULL;
        accf = (float*)calloc((size_t)N, sizeof(float));
        accd = (double*)calloc((size_t)N, sizeof(double));
        if (!accf || !accd) { free(accf); free(accd); break; }
        for (int g = 0; g < G; g++) {
            const int za = zero_int(A_zero[(int64_t)m * G + g]);
            const float sa = oracle_f16_to_f32(A_scale[(int64_t)m * G + g]);
            for (int n = 0; n < N; n++) P[n] = 0;
            const int k1 = (g + 1) * GROUP < K ? (g + 1) * GROUP : K;
            for (int k = g * GROUP; k < k1; k++) {
                const int32_t a = nib(arow, k) - za;
                const int32_t* vrow = vb + (int64_t)k * N;
                for (int n = 0; n < N; n++) P[n] += a * vrow[n];
            }
            for (int n = 0; n < N; n++) {
                const float sb = oracle_f16_to_f32(B_scale[(int64_t)g * N + n]);
                accf[n] = fmaf(sa * sb, (float)P[n], accf[n]);
                accd[n] += (double)sa * (double)sb * (double)P[n];
                if (partials) partials[((int64_t)m * N + n) * G + g] = P[n];
            }
        }
        for (int n = 0; n < N; n++) {
            if (C) C[(int64_t)m * N + n] = oracle_f32_to_f16(accf[n]);
            if (out64) out64[(int64_t)m * N + n] = accd[n];
        }
        free(accf);
        free(accd);
    }
    free(vb);
    free(P);
}

/*
 * W4A16 linear layer (fp16 activations x group-128 INT4 weights).  The
 * reference's runtime calls its linear layers through gemm_fp16 with an
 * optional beta=1 residual (src/runtime/inference.cu:139-194); the weight
 * format is gemm_int4's A operand (include/clove/kernels/gemm.cuh:74-87).
 */
void oracle_w4a16(const uint16_t* X, const uint8_t* W_q, const uint16_t* W_scale,
                  const uint16_t* W_zero, const uint16_t* Y_in, uint16_t* Y,
                  double* out64, int T, int O, int K, double alpha, double beta) {
    if (T <= 0 || O <= 0 || K <= 0) return;
    const int G = (K + GROUP - 1) / GROUP;
    const int half_k = K / 2;
    double* w = (double*)malloc((size_t)K * sizeof(double));
    double* x = (double*)malloc((size_t)K * T * sizeof(double));
    if (!w || !x) { free(w); free(x); return; }
    for (int64_t i = 0; i < (int64_t)T * K; i++) x[i] = (double)oracle_f16_to_f32(X[i]);
    for (int o = 0; o < O; o++) {
        const uint8_t* wrow = W_q + (int64_t)o * half_k;
        for (int k = 0; k < K; k++) {
            const int g = k / GROUP;
            const double s = (double)oracle_f16_to_f32(W_scale[(int64_t)o * G + g]);
            const int z = zero_int(W_zero[(int64_t)o * G + g]);
            w[k] = (double)(nib(wrow, k) - z) * s;
        }
        for (int t = 0; t < T; t++) {
            double acc = 0.0;
            const double* xr = x + (int64_t)t * K;
            for (int k = 0; k < K; k++) acc += xr[k] * w[k];
            double r = alpha * acc;
            const int64_t i = (int64_t)t * O + o;
            if (Y_in && beta != 0.0) r += beta * (double)oracle_f16_to_f32(Y_in[i]);
            if (out64) out64[i] = r;
            if (Y) Y[i] = oracle_f32_to_f16((float)r);
        }
    }
    free(w);
    free(x);
}

/*
 * SwiGLU on fp16 gate / up (src/kernels/activations.cu:9-11 silu_f,
 * :76-134 swiglu_kernel): out = fp16(silu(g) * u), g and u widened exactly
 * to fp32, silu(x) = x / (1 + expf(-x)) in fp32, the product rounded to fp32
 * and then to fp16 (__float2half of a float).
 */
void oracle_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float x = oracle_f16_to_f32(gate[i]);
        const float s = x / (1.0f + expf(-x));
        const float r = s * oracle_f16_to_f32(up[i]);
        out[i] = oracle_f32_to_f16(r);
    }
}
