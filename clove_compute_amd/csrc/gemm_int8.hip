// INT8 (W8A8) GEMM for gfx950.
//
//   acc[m,n] = sum_k (A_q[m,k] - za) * (B_q[k,n] - zb)      int32, exact
//   C[m,n]   = fp16(float(acc) * scale)   scale = A_scale*B_scale, or sa[m]*sb[n]
//
// Replaces the reference's gemm_int8 (src/kernels/gemm_int8.cu:16-137; the
// per-element formula is :37-40, :87-96, :113-114).
//
//  * int8_mfma -- v_mfma_i32_32x32x32_i8 on the raw operands.  Zero points are
//    applied exactly in the epilogue with the identity
//        sum (a-za)(b-zb) = sum ab - zb*rowsum(A) - za*colsum(B) + K*za*zb
//    (int32 wrap-around arithmetic, exact whenever the true value fits int32),
//    the row/column sums coming from a small pre-pass when a zero is non-zero.
//    B [K,N] is N-contiguous: each thread transposes 4 K rows x 16 columns of
//    bytes in registers (v_perm) on the way to LDS.
//  * int8_gemv -- M <= 4: B streamed once with 16-byte loads (a 256-column
//    tile per workgroup, all in flight), each column's four k rows
//    of a thread transposed into one dword (v_perm) for one v_dot4_i32_i8,
//    zero points by the same expansion, split-K over workgroups.
#include "common.hpp"
#include "dispatch.hpp"
#include "i8_dma_gemm.hpp"
#include "mfma_gemm.hpp"

namespace clove {
namespace i8 {

using namespace hw;

struct I8Params {
    const int8_t* A;
    const int8_t* B;
    void* C;
    const uint16_t* sa;
    const uint16_t* sb;
    const int* rowsum;  // [M] sum_k A (only when zb != 0)
    const int* colsum;  // [N] sum_k B (only when za != 0)
    float scale;
    int za, zb;
    int acc_add;  // added to every accumulator (int32 wrap-around): the
                  // reference-literal mode's padded-k term, else 0
    int M, N, K;
    int tiles_m, tiles_n, nsplit, k_per_split;
    float* ws;
    unsigned* counters;
};

// one output: int32 as is, or acc * s to fp16, s = sa[m] * sb[n] (loaded by
// the caller before its first store) for kHalfRowCol, else the tensor scale
template <int OUT>
__device__ __forceinline__ void int8_store(const I8Params& p, int m, int n, int acc, float s) {
    acc = (int)((unsigned)acc + (unsigned)p.acc_add);
    if constexpr (OUT == (int)Int8Out::kAcc32) {
        static_cast<int*>(p.C)[(int64_t)m * p.N + n] = acc;
    } else {
        if constexpr (OUT != (int)Int8Out::kHalfRowCol) s = p.scale;
        static_cast<uint16_t*>(p.C)[(int64_t)m * p.N + n] = f2h(static_cast<float>(acc) * s);
    }
}

// exact zero-point correction, int32 wrap-around arithmetic; rowsum = sum_k A of
// the output's row m, colsum = sum_k B of its column n
__device__ __forceinline__ int zero_correct(const I8Params& p, int acc, int rowsum, int colsum) {
    unsigned r = (unsigned)acc;
    if (p.zb != 0) r -= (unsigned)p.zb * (unsigned)rowsum;
    if (p.za != 0) r -= (unsigned)p.za * (unsigned)colsum;
    r += (unsigned)p.K * (unsigned)p.za * (unsigned)p.zb;
    return (int)r;
}

// ---------------------------------------------------------------------------
// pre-pass: row sums of A (one wave per row) and column sums of B
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) int8_rowsum(const int8_t* A, int M, int K, int* out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    int s = 0;
    for (int k = lane; k < K; k += 64) s += A[(int64_t)row * K + k];
    s = wave_sum(s);
    if (lane == 0) out[row] = s;
}

__global__ void __launch_bounds__(256) int8_colsum(const int8_t* B, int N, int K, int* out) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    int s = 0;
    for (int k = 0; k < K; ++k) s += B[(int64_t)k * N + n];
    out[n] = s;
}

// ---------------------------------------------------------------------------
// MFMA tile kernel
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WGM, int WGN, int OUT, bool ALIGNED>
__global__ void __launch_bounds__(WGM* WGN * 64) int8_mfma(I8Params p) {
    constexpr int NT = WGM * WGN * 64;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int LDK = BK + 16;  // bytes; 16-byte pad
    static_assert(BK % 32 == 0 && WTM % 32 == 0 && WTN % 32 == 0, "tile");
    constexpr int A_CH = BM * BK / 16;              // 16-byte chunks of A
    constexpr int LA = (A_CH + NT - 1) / NT;
    constexpr int B_BLK = (BK / 4) * (BN / 16);     // 4 K rows x 16 columns
    constexpr int LB = (B_BLK + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * LDK];
    __shared__ int s_last;

    mg::Params tp{};
    tp.tiles_m = p.tiles_m; tp.tiles_n = p.tiles_n; tp.nsplit = p.nsplit;
    const mg::TileCoord tc = mg::decode_tile(tp);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = tc.tm * BM, n0 = tc.tn * BN;
    const int M = p.M, N = p.N, K = p.K;
    const int kbeg = tc.split * p.k_per_split;
    const int kend = min(K, kbeg + p.k_per_split);
    const int ktiles = kend > kbeg ? cdiv(kend - kbeg, BK) : 0;

    unsigned ra[LA][4];
    unsigned rb[LB][4][4];

    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int c = tid + i * NT;
            const int row = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            const int gm = m0 + row, gk = k0 + kc;
            const bool in = (A_CH % NT == 0 || c < A_CH) && gm < M;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (in && gk < kend) v = *reinterpret_cast<const u32x4*>(p.A + (int64_t)gm * K + gk);
                ra[i][0] = v.x; ra[i][1] = v.y; ra[i][2] = v.z; ra[i][3] = v.w;
            } else {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    unsigned w = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int k = gk + 4 * d + e;
                        const unsigned b = (in && k < kend) ? (uint8_t)p.A[(int64_t)gm * K + k] : 0u;
                        w |= b << (8 * e);
                    }
                    ra[i][d] = w;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = tid + i * NT;
            const bool bin = B_BLK % NT == 0 || b < B_BLK;
            const int kb = b % (BK / 4), nb = b / (BK / 4);
            const int gn = n0 + nb * 16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gk = k0 + kb * 4 + r;
                if constexpr (ALIGNED) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (bin && gk < kend && gn < N) v = *reinterpret_cast<const u32x4*>(p.B + (int64_t)gk * N + gn);
                    rb[i][r][0] = v.x; rb[i][r][1] = v.y; rb[i][r][2] = v.z; rb[i][r][3] = v.w;
                } else {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        unsigned w = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int n = gn + 4 * d + e;
                            const unsigned bb = (bin && gk < kend && n < N) ? (uint8_t)p.B[(int64_t)gk * N + n] : 0u;
                            w |= bb << (8 * e);
                        }
                        rb[i][r][d] = w;
                    }
                }
            }
        }
    };

    auto store = [&](int st) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int c = tid + i * NT;
            if (A_CH % NT != 0 && c >= A_CH) continue;
            const int row = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            *reinterpret_cast<u32x4*>(&sA[st][row * LDK + kc]) = u32x4{ra[i][0], ra[i][1], ra[i][2], ra[i][3]};
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = tid + i * NT;
            if (B_BLK % NT != 0 && b >= B_BLK) continue;
            const int kb = b % (BK / 4), nb = b / (BK / 4);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                // 4x4 byte transpose of rows r=0..3, dword d -> columns 4d..4d+3
                const unsigned t0 = __builtin_amdgcn_perm(rb[i][1][d], rb[i][0][d], 0x05010400u);
                const unsigned t1 = __builtin_amdgcn_perm(rb[i][1][d], rb[i][0][d], 0x07030602u);
                const unsigned t2 = __builtin_amdgcn_perm(rb[i][3][d], rb[i][2][d], 0x05010400u);
                const unsigned t3 = __builtin_amdgcn_perm(rb[i][3][d], rb[i][2][d], 0x07030602u);
                const unsigned c0 = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
                const unsigned c1 = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
                const unsigned c2 = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
                const unsigned c3 = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
                int8_t* dst = &sB[st][(nb * 16 + 4 * d) * LDK + kb * 4];
                *reinterpret_cast<unsigned*>(dst) = c0;
                *reinterpret_cast<unsigned*>(dst + LDK) = c1;
                *reinterpret_cast<unsigned*>(dst + 2 * LDK) = c2;
                *reinterpret_cast<unsigned*>(dst + 3 * LDK) = c3;
            }
        }
    };

    i32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    if (ktiles > 0) {
        load(kbeg);
        store(0);
        __syncthreads();
    }
    const int lrow = lane & 31, lk = (lane >> 5) * 16;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load(kbeg + (kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            i32x4 bf[FN], af[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i)
                bf[i] = *reinterpret_cast<const i32x4*>(&sB[st][(wn * WTN + i * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int j = 0; j < FM; ++j)
                af[j] = *reinterpret_cast<const i32x4*>(&sA[st][(wm * WTM + j * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[i], af[j], acc[i][j], 0, 0, 0);
        }
        if (more) store(st ^ 1);
        __syncthreads();
    }

    if (p.nsplit > 1) {
        constexpr int NC = FN * FM * 4;  // 16-byte chunks of int32 partials per thread
        const int tile_id = tc.tm * p.tiles_n + tc.tn;
        float* slabs = p.ws + (int64_t)tile_id * p.nsplit * (BM * BN);
        f32x4 v[NC];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[(i * FM + j) * 4 + q] = bitcast<f32x4>(i32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                                                   acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
        splitk_publish<NC, NT>(slabs + (int64_t)tc.split * (BM * BN), tid, v);
        if (!splitk_arrive_is_last(&p.counters[tile_id], (unsigned)p.nsplit, &s_last)) return;
        splitk_reduce<NC, NT, true>(slabs, p.nsplit, tc.split, tid, v);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const i32x4 w = bitcast<i32x4>(v[(i * FM + j) * 4 + q]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = w[e];
                }
    }

    // the row / column factors of the lane's outputs first (clamped indices),
    // then the stores: a load issued after a store waits for it
    float rs[FM], cs[FN][16];
    int rsum[FM], csum[FN][16];
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int gm = min(m0 + wm * WTM + j * 32 + lrow, M - 1);
        rs[j] = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sa[gm]) : 1.0f;
        rsum[j] = p.zb != 0 ? p.rowsum[gm] : 0;
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int gn = min(n0 + wn * WTN + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), N - 1);
            cs[i][r] = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sb[gn]) : 1.0f;
            csum[i][r] = p.za != 0 ? p.colsum[gn] : 0;
        }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int gm = m0 + wm * WTM + j * 32 + lrow;
            if (gm >= M) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gn = n0 + wn * WTN + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (gn >= N) continue;
                int8_store<OUT>(p, gm, gn, zero_correct(p, acc[i][j][r], rsum[j], csum[i][r]), rs[j] * cs[i][r]);
            }
        }
}

// ---------------------------------------------------------------------------
// GEMV (M <= 4): 1024 threads = CL column lanes x (1024 / CL) K lanes; a
// column lane owns 16 consecutive columns (one 16-byte load per K row).
// ---------------------------------------------------------------------------
// A workgroup owns 256 columns x 256 k-rows of B (16 column lanes, 64 k
// lanes): thread (kl, cl) loads the 16 bytes of columns 16cl..16cl+15 of rows
// kl + 64 j, j < 4, so each wave instruction reads whole 256-byte row segments
// and the workgroup's 64 KB tile is requested at once (4096 x 4096: 256
// workgroups).  Measured on 4096 x 4096 with the one-round-trip split-K below:
// M = 1 at 128 / 256 / 512 columns 6.43 / 5.92 / 5.90 us, M = 2 at 128 / 256
// columns 7.47 / 6.95 us.  Loads are unconditional from clamped addresses
// (masked at use).  int32 sums: within a wave (v_permlane row swaps), across
// the 16 waves through LDS, then across the K splits (one round trip, see the
// end of the kernel).
constexpr int kIvCols = 256, kIvKl = 1024 / (kIvCols / 16), kIvRpt = 4, kIvRows = kIvKl * kIvRpt;

template <int MM, int OUT>
__global__ void __launch_bounds__(1024) int8_gemv(I8Params p, int col_blocks) {
    constexpr int IV_RPT = kIvRpt, IV_ROWS = kIvRows;
    constexpr int IV_COLS = kIvCols, IV_KL = kIvKl, CL = IV_COLS / 16;  // CL: column lanes
    __shared__ __attribute__((aligned(16))) int red[16][MM][IV_COLS];
    static_assert(CL == 16, "column lanes");
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int cl = tid % CL, kl = tid / CL, wave = tid >> 6, lane = tid & 63;
    const int split = blockIdx.x % p.nsplit;
    const int cb = blockIdx.x / p.nsplit;
    const int M = p.M, N = p.N, K = p.K;
    const int n = cb * IV_COLS + cl * 16;
    const int nc = min(n, N - 16);
    const int kbeg = split * IV_ROWS;

    // A first (see gemv_f16): the products of row j then wait only for B row j
    int8_t xa[MM][IV_RPT];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int j = 0; j < IV_RPT; ++j)
            xa[m][j] = p.A[(int64_t)min(m, M - 1) * K + min(kbeg + kl + IV_KL * j, K - 1)];
    // (kept ahead of the B loads: one A load scheduled after them would make
    // the first product wait for every B row, loads completing in order)
    __builtin_amdgcn_sched_barrier(0);
    u32x4 bv[IV_RPT];
#pragma unroll
    for (int j = 0; j < IV_RPT; ++j) {
        const int k = min(kbeg + kl + IV_KL * j, K - 1);
        bv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.B + (int64_t)k * N + nc));
    }
    __builtin_amdgcn_sched_barrier(0);  // every B row requested before the first product

    // Each column's four k rows (k = kbeg + kl + IV_KL j, j < 4) in one dword:
    // a 4 x 4 byte transpose of the rows' 16-byte loads (v_perm), so that one
    // v_dot4_i32_i8 forms a column's four products and their sum.  Zero points
    // by  sum (a - za)(b - zb) = sum ab - za sum b - zb sum (a - za)  over the
    // valid rows (int32, exact: every term is small).  Rows past K (loaded from
    // the clamped last row) take a zero byte of A and of the row mask.
    static_assert(IV_RPT == 4, "one dot4 per column covers a thread's four rows");
    unsigned bc[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const unsigned lo01 = __builtin_amdgcn_perm(bv[1][c], bv[0][c], 0x05010400u);
        const unsigned hi01 = __builtin_amdgcn_perm(bv[1][c], bv[0][c], 0x07030602u);
        const unsigned lo23 = __builtin_amdgcn_perm(bv[3][c], bv[2][c], 0x05010400u);
        const unsigned hi23 = __builtin_amdgcn_perm(bv[3][c], bv[2][c], 0x07030602u);
        bc[4 * c] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);      // rows 0-3 of column 4c
        bc[4 * c + 1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);  // column 4c + 1
        bc[4 * c + 2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
        bc[4 * c + 3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
    unsigned ok4 = 0;  // byte j: 1 when row j lies inside K
    int nok = 0;
#pragma unroll
    for (int j = 0; j < IV_RPT; ++j)
        if (kbeg + kl + IV_KL * j < K) {
            ok4 |= 1u << (8 * j);
            ++nok;
        }

    // Rows of A in passes of at most two: the 16 column accumulators of four
    // rows would not fit beside the loads in flight.
    constexpr int MC = MM >= 4 ? 2 : MM;
#pragma unroll
    for (int m0 = 0; m0 < MM; m0 += MC) {
        int acc[MC][16];
#pragma unroll
        for (int m = 0; m < MC; ++m) {
            const bool in_m = m0 + m < M;
            unsigned ap = 0;  // byte j: row j's A value (zero past K or past M)
            int asum = 0;
#pragma unroll
            for (int j = 0; j < IV_RPT; ++j) {
                const int av = (in_m && kbeg + kl + IV_KL * j < K) ? (int)xa[m0 + m][j] : 0;
                ap |= ((unsigned)av & 0xffu) << (8 * j);
                asum += av;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[m][e] = __builtin_amdgcn_sdot4((int)ap, (int)bc[e], 0, false);
            if (p.za != 0) {
                const int mk = in_m ? (int)ok4 : 0;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[m][e] -= p.za * __builtin_amdgcn_sdot4(mk, (int)bc[e], 0, false);
            }
            if (p.zb != 0) {
                const int t = in_m ? asum - p.za * nok : 0;  // sum of (a - za) over the valid rows
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[m][e] -= p.zb * t;
            }
        }
        // the k lanes of a column lane are lanes l, l+16, l+32, l+48: row
        // swaps leave lane l of row r with column 16 cl + 4 u + r, u < 4
#pragma unroll
        for (int m = 0; m < MC; ++m)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                red[wave][m0 + m][cl * 16 + 4 * u + (lane >> 4)] =
                    rows_sum4(acc[m][4 * u], acc[m][4 * u + 1], acc[m][4 * u + 2], acc[m][4 * u + 3]);
    }
    __syncthreads();
    // threads 0..IV_COLS-1 own one column each from here on; every thread still
    // takes part in the arrival barrier
    const bool active = tid < IV_COLS;
    const int col = active ? tid : 0;
    const int gn = cb * IV_COLS + col;
    int sum[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        int s = 0;
#pragma unroll
        for (int q = 0; q < 16; ++q) s += red[q][m][col];
        sum[m] = s;
    }
    if (p.nsplit > 1 && p.ws == nullptr) {
        // one round trip: every split adds (1 << 48) + (sum + 2^31) to the
        // output's 64-bit word in the zeroed counter region with one
        // device-scope atomic; the split whose returned count is nsplit - 1
        // holds the whole exact integer sum (the low 48 bits, less nsplit 2^31),
        // stores the output and re-arms the word to zero for the next launch
        if (!active || gn >= N) return;
        const float cs = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sb[gn]) : 1.0f;
        uint64_t* acc64 = reinterpret_cast<uint64_t*>(p.counters) + (int64_t)cb * MM * IV_COLS + col;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (m >= M) break;
            const float rs = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sa[m]) : 1.0f;
            constexpr uint64_t kLow = ((uint64_t)1 << 48) - 1;
            const uint64_t add = ((uint64_t)1 << 48) | (uint64_t)((int64_t)sum[m] + 0x80000000ll);
            const uint64_t old = __hip_atomic_fetch_add(acc64 + m * IV_COLS, add, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            if ((old >> 48) == (uint64_t)(p.nsplit - 1)) {
                const int64_t tot = (int64_t)((old & kLow) + (add & kLow)) - (int64_t)p.nsplit * 0x80000000ll;
                __hip_atomic_store(acc64 + m * IV_COLS, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                int8_store<OUT>(p, m, gn, (int)(uint32_t)(uint64_t)tot, rs * cs);
            }
        }
        return;
    }
    if (p.nsplit > 1) {
        float* ws_tile = p.ws + (int64_t)cb * p.nsplit * (MM * IV_COLS);
        if (active) {
#pragma unroll
            for (int m = 0; m < MM; ++m)
                store_coherent(&ws_tile[(int64_t)split * MM * IV_COLS + m * IV_COLS + col], __int_as_float(sum[m]));
        }
        if (!splitk_arrive_is_last(&p.counters[cb], (unsigned)p.nsplit, &s_last)) return;
#pragma unroll
        for (int m = 0; m < MM; ++m) sum[m] = 0;
        // up to SB partials in flight together; none loaded past the last
        // split (the extra coherent loads lengthen the tail measurably)
        constexpr int SB = MM >= 4 ? 8 : 16;
        for (int s0 = 0; s0 < p.nsplit; s0 += SB) {
            int part[SB][MM];
#pragma unroll
            for (int s = 0; s < SB; ++s)
#pragma unroll
                for (int m = 0; m < MM; ++m)
                    part[s][m] = s0 + s < p.nsplit
                                     ? __float_as_int(load_coherent(
                                           &ws_tile[(int64_t)(s0 + s) * MM * IV_COLS + m * IV_COLS + col]))
                                     : 0;
#pragma unroll
            for (int s = 0; s < SB; ++s)
#pragma unroll
                for (int m = 0; m < MM; ++m) sum[m] += part[s][m];
        }
    }
    if (active && gn < N) {
        // every scale the stores use is loaded before the first store
        float rs[MM];
        const float cs = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sb[gn]) : 1.0f;
#pragma unroll
        for (int m = 0; m < MM; ++m)
            rs[m] = OUT == (int)Int8Out::kHalfRowCol ? h2f(p.sa[min(m, M - 1)]) : 1.0f;
#pragma unroll
        for (int m = 0; m < MM; ++m)
            if (m < M) int8_store<OUT>(p, m, gn, sum[m], rs[m] * cs);
    }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
namespace {

template <int OUT>
clove_status_t run_gemv(I8Params p, hipStream_t stream) {
    const int mm = p.M == 1 ? 1 : (p.M == 2 ? 2 : 4);
    const int rows = kIvRows;
    const int IV_COLS = kIvCols;
    const int col_blocks = cdiv(p.N, IV_COLS);
    p.nsplit = cdiv(p.K, rows);
    p.k_per_split = rows;
    p.ws = nullptr;
    p.counters = nullptr;
    if (p.nsplit > 1) {
        // the one-round-trip reduction needs one zeroed 64-bit word per output
        // (mm x IV_COLS per column block) in the counter region; a bound workspace
        // whose counter region is smaller takes the partial-tile reduction
        Scratch s;
        clove_status_t st = CLOVE_ERR_WORKSPACE;
        if (p.nsplit < 65536) st = acquire_scratch(stream, 0, (size_t)col_blocks * mm * IV_COLS * 2, &s);
        if (st == CLOVE_OK) {
            p.counters = s.counters;
        } else if (st == CLOVE_ERR_WORKSPACE) {
            st = acquire_scratch(stream, (size_t)col_blocks * p.nsplit * mm * IV_COLS * 4, (size_t)col_blocks, &s);
            if (st != CLOVE_OK) return st;
            p.ws = s.partials;
            p.counters = s.counters;
        } else {
            return st;
        }
    }
    const int64_t g = (int64_t)col_blocks * p.nsplit;
    if (g > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    const dim3 grid((unsigned)g);
    if (p.M == 1) CLOVE_LAUNCH((int8_gemv<1, OUT>), grid, dim3(1024), 0, stream, p, col_blocks);
    else if (p.M == 2) CLOVE_LAUNCH((int8_gemv<2, OUT>), grid, dim3(1024), 0, stream, p, col_blocks);
    else CLOVE_LAUNCH((int8_gemv<4, OUT>), grid, dim3(1024), 0, stream, p, col_blocks);
    return check_launch();
}

template <int BM, int BN, int BK, int WGM, int WGN, int OUT, bool ALIGNED>
clove_status_t run_mfma(I8Params p, int cus, hipStream_t stream) {
    p.tiles_m = cdiv(p.M, BM);
    p.tiles_n = cdiv(p.N, BN);
    const int tiles = p.tiles_m * p.tiles_n;
    const mg::SplitPlan sp = mg::plan_split(tiles, p.K, BK, cus, 2 * cus, 2);
    p.nsplit = sp.nsplit;
    p.k_per_split = sp.k_per_split;
    const bool sums = (p.za != 0 || p.zb != 0) && p.K > 0;
    const size_t part = p.nsplit > 1 ? (size_t)tiles * p.nsplit * BM * BN * 4 : 0;
    const size_t aux = sums ? ((size_t)p.M + p.N) * sizeof(int) : 0;
    if (part + aux > 0) {
        // one scratch request: split-K partials first, then the zero-point sums
        Scratch s;
        clove_status_t st = acquire_scratch(stream, part + aux, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
        if (sums) {
            int* rs = reinterpret_cast<int*>(reinterpret_cast<char*>(s.partials) + part);
            int* cs = rs + p.M;
            CLOVE_LAUNCH(int8_rowsum, dim3(cdiv(p.M, 4)), dim3(256), 0, stream, p.A, p.M, p.K, rs);
            CLOVE_LAUNCH(int8_colsum, dim3(cdiv(p.N, 256)), dim3(256), 0, stream, p.B, p.N, p.K, cs);
            p.rowsum = rs;
            p.colsum = cs;
        }
    }
    CLOVE_LAUNCH((int8_mfma<BM, BN, BK, WGM, WGN, OUT, ALIGNED>), dim3(tiles * p.nsplit),
                       dim3(WGM * WGN * 64), 0, stream, p);
    return check_launch();
}

// the 256x256 LDS-DMA kernel (i8_dma_gemm.hpp): zero points 0, K % 128 == 0,
// N % 16 == 0, 16-byte aligned operands under 2^31 bytes
bool i8big_eligible(const I8Params& p) {
    return p.za == 0 && p.zb == 0 && p.K > 0 && p.K % i8big::Cfg::BKB == 0 && p.N >= 16 && p.N % 16 == 0 &&
           aligned16(p.A) && aligned16(p.B) && aligned16(p.C) && (int64_t)p.M * p.K < (1ll << 31) &&
           (int64_t)p.K * p.N < (1ll << 31) && (int64_t)p.M * p.N * 4 < (1ll << 31);
}

template <int OUT>
clove_status_t run_i8big(const I8Params& q, hipStream_t stream) {
    i8big::Args a{};
    a.A = q.A;
    a.B = q.B;
    a.C = q.C;
    a.sa = q.sa;
    a.sb = q.sb;
    a.scale = q.scale;
    a.M = q.M;
    a.N = q.N;
    a.K = q.K;
    a.tiles_m = cdiv(q.M, i8big::Cfg::BM);
    a.tiles_n = cdiv(q.N, i8big::Cfg::BN);
    constexpr int KO = OUT == (int)Int8Out::kAcc32       ? (int)i8big::kAcc32
                       : OUT == (int)Int8Out::kHalfRowCol ? (int)i8big::kRowCol
                                                          : (int)i8big::kTensor;
    CLOVE_LAUNCH((i8big::gemm_i8_big<KO>), dim3((unsigned)(a.tiles_m * a.tiles_n)), dim3(i8big::Cfg::NT), 0,
                 stream, a);
    return check_launch();
}

template <int OUT>
clove_status_t dispatch(I8Params p, bool aligned, int cus, hipStream_t stream) {
    if (aligned && p.M <= 4 && p.K > 0 && p.N >= 16) return run_gemv<OUT>(p, stream);
    if (!aligned) return run_mfma<64, 64, 64, 2, 2, OUT, false>(p, cus, stream);
    if (p.M <= 64) return run_mfma<64, 128, 128, 2, 2, OUT, true>(p, cus, stream);
    if ((int64_t)cdiv(p.M, 256) * cdiv(p.N, 256) >= cus / 2)
        return run_mfma<256, 256, 64, 2, 2, OUT, true>(p, cus, stream);
    return run_mfma<128, 128, 128, 2, 2, OUT, true>(p, cus, stream);
}

}  // namespace
}  // namespace i8

clove_status_t launch_gemm_int8(const Int8Args& a, hipStream_t stream) {
    using namespace i8;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    I8Params p{};
    p.A = a.A; p.B = a.B; p.C = a.C; p.sa = a.sa; p.sb = a.sb;
    p.scale = a.scale; p.za = a.za; p.zb = a.zb; p.acc_add = a.acc_add;
    p.M = a.M; p.N = a.N; p.K = a.K;
    const bool aligned = aligned16(a.A) && aligned16(a.B) && (a.K % 16 == 0) && (a.N % 16 == 0);
    // 256x256 tiles once they cover half the CUs (cold weights, against the
    // skinny kernel: 4096^3 146.5 -> 64.1 us, 11008x4096 at M = 768 94.2 ->
    // 50.2 us, 8192x8192 at M = 1024 153.3 -> 86.1 us; with fewer tiles the
    // skinny kernel is ahead: 4096x4096 at M = 1024 43.9 against 60.1 us)
    if ((int64_t)cdiv(a.M, i8big::Cfg::BM) * cdiv(a.N, i8big::Cfg::BN) >= dev.num_cus / 2 && i8big_eligible(p)) {
        switch (a.out) {
            case Int8Out::kHalfPerTensor: return run_i8big<(int)Int8Out::kHalfPerTensor>(p, stream);
            case Int8Out::kHalfRowCol: return run_i8big<(int)Int8Out::kHalfRowCol>(p, stream);
            case Int8Out::kAcc32: return run_i8big<(int)Int8Out::kAcc32>(p, stream);
        }
    }
    if (a.M > 2) {  // (three or four rows only for large weights; try_skinny_int8 decides)
        clove_status_t st2;
        if (try_skinny_int8(a, dev.num_cus, stream, &st2)) return st2;
    }
    switch (a.out) {
        case Int8Out::kHalfPerTensor: return dispatch<(int)Int8Out::kHalfPerTensor>(p, aligned, dev.num_cus, stream);
        case Int8Out::kHalfRowCol: return dispatch<(int)Int8Out::kHalfRowCol>(p, aligned, dev.num_cus, stream);
        case Int8Out::kAcc32: return dispatch<(int)Int8Out::kAcc32>(p, aligned, dev.num_cus, stream);
    }
    return CLOVE_ERR_INVALID_ARG;
}

}  // namespace clove
