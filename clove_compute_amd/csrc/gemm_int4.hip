// Packed INT4 x INT4 GEMM (gemm_int4) for gfx950.
//
// Replaces the reference's gemm_int4 (src/kernels/gemm_int4.cu:45-216).
// Layouts (include/clove/kernels/gemm.cuh:74-87): A_q [M, K/2] with the even k
// in the high nibble; B_q [K, ceil(N/2)] packed along N, even n in the high
// nibble; scales/zeros [M, G] and [G, N], G = ceil(K/128).
//
//  * int4_gemv (N <= 8, the decode shapes) -- one group of LPR lanes streams
//    one weight row with 16-byte loads (32 nibbles per lane per step).  The
//    per-group integer partials are exact:
//       P = sum qA*qB - zB*sum qA - zA*sum qB + cnt*zA*zB
//    with sum qA*qB from v_dot8_u32_u4 on nibble words, the B words (in A's
//    nibble order) and their chunk sums staged once per workgroup in LDS.
//    Group-wise: acc += (sA*sB) * float(P) per 32-k chunk, fp32.
//    Literal: int32 S accumulates sum (qA-8)(qB-8) over all K.
//  * larger N -- the shared MFMA GEMM (mfma_gemm.hpp) with INT4 loaders that
//    unpack both operands to the exact integers q - z in fp16 on their way to
//    LDS; per-group fp32 partials (exact) are scaled by sA*sB after each
//    128-wide group.
#include "common.hpp"
#include "dispatch.hpp"
#include "mfma_gemm.hpp"

#include <type_traits>

namespace clove {
namespace i4 {

using namespace hw;

struct GemvParams {
    const uint8_t* A;
    const uint16_t* A_scale;
    const uint16_t* A_zero;
    const uint8_t* B;
    const uint16_t* B_scale;
    const uint16_t* B_zero;
    uint16_t* C;
    int M, N, K, G;
    int ldb;          // bytes per K row of B
    int cols_valid;   // columns n >= cols_valid read no B (literal: 2*floor(N/2))
    int nch;          // 32-k chunks per row = ceil(K/32)
};

constexpr unsigned kOnes = 0x11111111u;  // eight 4-bit ones

__global__ void fill_u16(uint16_t* p, size_t n, uint16_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// LDS layout (dynamic): raw B bytes [K * ldb] (staging, rounded up to 16 bytes) |
// Bw [NV][4*nch] u32 | Bsum [NV][nch] int | Bs [NV][G] f32 | Bz [NV][G] int
__host__ __device__ inline size_t gemv_lds_bytes(int nv, int nch, int G, int K, int ldb) {
    return (size_t)nv * ((size_t)4 * nch * 4 + (size_t)nch * 4 + (size_t)G * 8) +
           (((size_t)K * ldb + 15) & ~(size_t)15);
}

template <int NV, int MODE, int LPR, bool ALIGNED>
__global__ void __launch_bounds__(256) int4_gemv(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned lds[];
    constexpr int RPW = 256 / LPR;  // rows per workgroup
    constexpr int UNR = 4;          // chunks in flight per lane
    const int tid = threadIdx.x;
    const int nch = p.nch, K = p.K, G = p.G;
    const int KWP = 4 * nch;
    // raw bytes first so both the 16-byte staging stores and Bw stay aligned
    uint8_t* Braw = reinterpret_cast<uint8_t*>(lds);
    const int rawsz = p.cols_valid > 0 ? ((K * p.ldb + 15) & ~15) : 0;
    unsigned* Bw = reinterpret_cast<unsigned*>(Braw + rawsz);
    int* Bsum = reinterpret_cast<int*>(Bw + NV * KWP);
    float* Bs = reinterpret_cast<float*>(Bsum + NV * nch);
    int* Bz = reinterpret_cast<int*>(Bs + NV * G);

    const int row = blockIdx.x * RPW + tid / LPR;
    const int lr = tid % LPR;
    const bool row_ok = row < p.M;
    const uint8_t* arow = p.A + (int64_t)row * (K / 2);

    // ---- prefetch the first batch of A chunks (overlaps the B staging) ----
    unsigned a_cur[UNR][4];
    uint16_t s_cur[UNR], z_cur[UNR];
    auto load_batch = [&](int c0, unsigned (&a)[UNR][4], uint16_t (&s)[UNR], uint16_t (&z)[UNR]) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int c = c0 + u * LPR;
            const bool in = row_ok && c < nch;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (in) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(arow + 16 * c));
                a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
            } else {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    unsigned w = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int byte = 16 * c + 4 * d + e;
                        const unsigned b = (in && 2 * byte < K) ? arow[byte] : 0u;
                        w |= b << (8 * e);
                    }
                    a[u][d] = w;
                }
            }
            if constexpr (MODE == mg::kI4Groupwise) {
                const int64_t gi = (int64_t)row * G + (c >> 2);
                s[u] = in ? p.A_scale[gi] : (uint16_t)0;
                z[u] = in ? p.A_zero[gi] : (uint16_t)0;
            }
        }
    };
    load_batch(lr, a_cur, s_cur, z_cur);

    // ---- stage B: raw bytes (16-byte loads), then nibble words in A's order ----
    const int braw = p.cols_valid > 0 ? K * p.ldb : 0;
    if ((reinterpret_cast<uintptr_t>(p.B) & 15) == 0) {
        for (int i = tid; 16 * i < braw; i += 256) {
            if (16 * i + 16 <= braw) {
                *reinterpret_cast<u32x4*>(Braw + 16 * i) = *reinterpret_cast<const u32x4*>(p.B + 16 * i);
            } else {
                for (int j = 16 * i; j < braw; ++j) Braw[j] = p.B[j];
            }
        }
    } else {
        for (int i = tid; i < braw; i += 256) Braw[i] = p.B[i];
    }
    __syncthreads();
    for (int idx = tid; idx < NV * KWP; idx += 256) {
        const int n = idx / KWP, w = idx - n * KWP;
        unsigned word = 0;
        if (n < p.cols_valid) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int k = 8 * w + j;
                if (k < K) {
                    const unsigned byte = Braw[k * p.ldb + (n >> 1)];
                    const unsigned nib = (n & 1) ? (byte & 0xfu) : (byte >> 4);
                    word |= nib << (8 * (j >> 1) + ((j & 1) ? 0 : 4));
                }
            }
        }
        Bw[idx] = word;
    }
    if constexpr (MODE == mg::kI4Groupwise) {
        for (int idx = tid; idx < NV * G; idx += 256) {
            const int n = idx / G, g = idx - n * G;
            const bool in = n < p.N;
            Bs[idx] = in ? h2f(p.B_scale[(int64_t)g * p.N + n]) : 0.0f;
            Bz[idx] = in ? (int)rintf(h2f(p.B_zero[(int64_t)g * p.N + n])) : 0;
        }
    }
    __syncthreads();
    for (int idx = tid; idx < NV * nch; idx += 256) {
        const int n = idx / nch, c = idx - n * nch;
        const unsigned* bw = Bw + n * KWP + 4 * c;
        unsigned s = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) s = __builtin_amdgcn_udot8(bw[d], kOnes, s, false);
        Bsum[idx] = (int)s;
    }
    __syncthreads();

    // ---- stream the row ----
    float accf[NV];
    int acci[NV];
#pragma unroll
    for (int n = 0; n < NV; ++n) { accf[n] = 0.0f; acci[n] = 0; }

    for (int c0 = lr; c0 < nch; c0 += UNR * LPR) {
        unsigned a_nxt[UNR][4];
        uint16_t s_nxt[UNR], z_nxt[UNR];
        const bool more = c0 + UNR * LPR < nch;
        if (more) load_batch(c0 + UNR * LPR, a_nxt, s_nxt, z_nxt);
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int c = c0 + u * LPR;
            if (c >= nch) break;
            const int g = c >> 2;
            const int cnt = min(32, K - 32 * c);
            unsigned sa = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) sa = __builtin_amdgcn_udot8(a_cur[u][d], kOnes, sa, false);
            int za = 0;
            float fa = 0.0f;
            if constexpr (MODE == mg::kI4Groupwise) {
                za = (int)rintf(h2f(z_cur[u]));
                fa = h2f(s_cur[u]);
            }
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                const u32x4 bw = *reinterpret_cast<const u32x4*>(Bw + n * KWP + 4 * c);
                unsigned dot = __builtin_amdgcn_udot8(a_cur[u][0], bw.x, 0u, false);
                dot = __builtin_amdgcn_udot8(a_cur[u][1], bw.y, dot, false);
                dot = __builtin_amdgcn_udot8(a_cur[u][2], bw.z, dot, false);
                dot = __builtin_amdgcn_udot8(a_cur[u][3], bw.w, dot, false);
                const int sb = Bsum[n * nch + c];
                if constexpr (MODE == mg::kI4Groupwise) {
                    const int zb = Bz[n * G + g];
                    const int P = (int)dot - zb * (int)sa - za * sb + cnt * za * zb;
                    accf[n] = fmaf(fa * Bs[n * G + g], (float)P, accf[n]);
                } else {
                    if (n < p.cols_valid) acci[n] += (int)dot - 8 * (int)sa - 8 * sb + 64 * cnt;
                }
            }
        }
        if (more) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
#pragma unroll
                for (int d = 0; d < 4; ++d) a_cur[u][d] = a_nxt[u][d];
                s_cur[u] = s_nxt[u];
                z_cur[u] = z_nxt[u];
            }
        }
    }

    // ---- reduce over the LPR lanes of the row (fixed butterfly order) ----
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            if constexpr (MODE == mg::kI4Groupwise) accf[n] += __shfl_xor(accf[n], off);
            else acci[n] += __shfl_xor(acci[n], off);
        }
    }
    if (row_ok && lr == 0) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            if (n >= p.N) break;
            float r;
            if constexpr (MODE == mg::kI4Groupwise) {
                r = accf[n];
            } else {
                const float a_s = h2f(p.A_scale[(int64_t)row * G + (G - 1)]);
                const float b_s = h2f(p.B_scale[(int64_t)(G - 1) * p.N + n]);
                r = ((float)acci[n] * a_s) * b_s;
            }
            p.C[(int64_t)row * p.N + n] = f2h(r);
        }
    }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kMaxGemvLds = 150 * 1024;

template <int NV, int MODE>
clove_status_t run_gemv(const GemvParams& p, bool aligned, hipStream_t stream) {
    constexpr int LPR = 16;
    const size_t lds = gemv_lds_bytes(NV, p.nch, p.G, p.K, p.ldb);
    const dim3 grid(cdiv(p.M, 256 / LPR));
    if (aligned) {
        auto k = int4_gemv<NV, MODE, LPR, true>;
        if (lds > 64 * 1024 &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return CLOVE_ERR_LAUNCH;
        hipLaunchKernelGGL(k, grid, dim3(256), lds, stream, p);
    } else {
        auto k = int4_gemv<NV, MODE, LPR, false>;
        if (lds > 64 * 1024 &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return CLOVE_ERR_LAUNCH;
        hipLaunchKernelGGL(k, grid, dim3(256), lds, stream, p);
    }
    return check_launch();
}

template <int MODE>
clove_status_t gemv_by_n(const GemvParams& p, bool aligned, hipStream_t stream) {
    if (p.N == 1) return run_gemv<1, MODE>(p, aligned, stream);
    if (p.N == 2) return run_gemv<2, MODE>(p, aligned, stream);
    if (p.N <= 4) return run_gemv<4, MODE>(p, aligned, stream);
    return run_gemv<8, MODE>(p, aligned, stream);
}

using mg::Tile;

template <class T, int MODE, bool ALIGNED>
clove_status_t run_mfma(mg::Params p, int cus, hipStream_t stream) {
    using LA = mg::LoadI4Rows<T::BM, T::BK, T::NT, T::LDK, false, MODE, ALIGNED>;
    using LB = mg::LoadI4Cols<T::BN, T::BK, T::NT, T::LDK, MODE, ALIGNED>;
    using EPI = typename std::conditional<MODE == mg::kI4Literal, mg::EpiI4Literal,
                                          mg::EpiAlphaBeta<false>>::type;
    p.tiles_m = cdiv(p.M, T::BM);
    p.tiles_n = cdiv(p.N, T::BN);
    const int tiles = p.tiles_m * p.tiles_n;
    // splits on 128-wide group boundaries so every group is folded whole
    const mg::SplitPlan sp = mg::plan_split(tiles, p.K, 128, cus, 2 * cus, 2);
    p.nsplit = sp.nsplit;
    p.k_per_split = sp.k_per_split;
    if (p.nsplit > 1) {
        Scratch s;
        clove_status_t st = acquire_scratch(stream, (size_t)tiles * p.nsplit * T::BM * T::BN * 4,
                                            (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
    }
    constexpr int FOLD = MODE == mg::kI4Literal ? mg::kFoldNone : mg::kFoldAB;
    hipLaunchKernelGGL((mg::mfma_gemm<T, LA, LB, EPI, FOLD>), dim3(tiles * p.nsplit), dim3(T::NT), 0,
                       stream, p);
    return check_launch();
}

template <int MODE>
clove_status_t mfma_by_shape(const mg::Params& p, bool aligned, int cus, hipStream_t stream) {
    if (!aligned) return run_mfma<Tile<64, 64, 64, 2, 2>, MODE, false>(p, cus, stream);
    if (p.N <= 32) return run_mfma<Tile<128, 32, 64, 4, 1>, MODE, true>(p, cus, stream);
    if (p.N <= 64) return run_mfma<Tile<128, 64, 64, 2, 2>, MODE, true>(p, cus, stream);
    return run_mfma<Tile<64, 128, 64, 2, 2>, MODE, true>(p, cus, stream);
}

}  // namespace
}  // namespace i4

clove_status_t launch_gemm_int4(const Int4Args& a, hipStream_t stream) {
    using namespace i4;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const bool literal = a.mode == CLOVE_INT4_REFERENCE_LITERAL;
    const int G = cdiv(a.K, 128);
    const int ldb = literal ? a.N / 2 : (a.N + 1) / 2;
    const int cols_valid = literal ? 2 * (a.N / 2) : a.N;
    const int nch = cdiv(a.K, 32);
    if (a.K == 0) {
        // empty sum: +0 in both modes (the reference reads no scale group then)
        const size_t n = (size_t)a.M * a.N;
        hipLaunchKernelGGL(fill_u16, dim3((unsigned)(n < 1048576 ? cdiv64(n, 256) : 4096)), dim3(256), 0,
                           stream, a.C, n, (uint16_t)0);
        return check_launch();
    }
    if (a.N <= 8 && gemv_lds_bytes(a.N <= 2 ? a.N : (a.N <= 4 ? 4 : 8), nch, G, a.K, ldb) <= kMaxGemvLds) {
        GemvParams p{a.A, a.A_scale, a.A_zero, a.B, a.B_scale, a.B_zero, a.C,
                     a.M, a.N, a.K, G, ldb, cols_valid, nch};
        const bool aligned = aligned16(a.A) && (a.K % 32 == 0);
        return literal ? gemv_by_n<mg::kI4Literal>(p, aligned, stream)
                       : gemv_by_n<mg::kI4Groupwise>(p, aligned, stream);
    }
    mg::Params p{};
    p.a = a.A; p.a_scale = a.A_scale; p.a_zero = a.A_zero;
    p.b = a.B; p.b_scale = a.B_scale; p.b_zero = a.B_zero;
    p.c = a.C;
    p.M = a.M; p.N = a.N; p.K = a.K; p.G = G;
    p.ldb_bytes = ldb;
    p.b_cols_valid = cols_valid;
    p.alpha = 1.0f; p.beta = 0.0f;
    const bool aligned = aligned16(a.A) && (a.K % 32 == 0) && (reinterpret_cast<uintptr_t>(a.B) % 8 == 0) &&
                         (ldb % 8 == 0);
    return literal ? mfma_by_shape<mg::kI4Literal>(p, aligned, dev.num_cus, stream)
                   : mfma_by_shape<mg::kI4Groupwise>(p, aligned, dev.num_cus, stream);
}

}  // namespace clove
