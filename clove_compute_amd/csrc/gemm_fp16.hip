// FP16 GEMM for gfx950: C = alpha * A @ B + beta * C, fp32 accumulation.
//
// Replaces the reference's gemm_fp16 (src/kernels/gemm_fp16.cu:277-305) and
// gemm_fp16_batched (:366-383).  Two kernels:
//
//  * gemm_f16_mfma  -- LDS-tiled v_mfma_f32_32x32x16_f16 GEMM, double-buffered
//    LDS, register-staged global loads (16 B per lane), optional split-K with a
//    deterministic last-arriver reduction.  B [K,N] is N-contiguous; each lane
//    transposes an 8x8 (or 4x8) half block in registers on its way to LDS so
//    both operands sit K-contiguous in LDS and every fragment is one
//    ds_read_b128.
//  * gemv_f16       -- M <= 4 decode shapes: B streamed once from HBM with
//    16 B loads, fp32 FMAs on the VALU, split-K over workgroups.
#include "common.hpp"
#include "dispatch.hpp"

namespace clove {
namespace fp16 {

using namespace hw;

struct GemmParams {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    int M, N, K;
    float alpha, beta;
    int64_t strideA, strideB, strideC;  // elements between batches
    int tiles_m, tiles_n;
    int nsplit;       // workgroups along K per output tile
    int k_per_split;  // multiple of the K tile
    float* ws;        // split-K partials
    unsigned* counters;
};

__device__ __forceinline__ f16x8 lds_read_f16x8(const uint16_t* p) {
    return bitcast<f16x8>(*reinterpret_cast<const u32x4*>(p));
}

// Workgroup id -> (batch, tile_m, tile_n, split).  Workgroups are handed to the
// 8 XCDs round-robin; when the grid divides by 8 the id is first permuted so
// that each XCD owns a contiguous range of logical tiles, and logical tiles are
// walked in column groups of 8 tile-rows, so one XCD's workgroups share A and
// B panels in its L2.
struct TileCoord {
    int batch, tm, tn, split;
};
__device__ __forceinline__ TileCoord decode_tile(const GemmParams& p) {
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    TileCoord t;
    t.split = bid % p.nsplit;
    int tile = bid / p.nsplit;
    const int per_batch = p.tiles_m * p.tiles_n;
    t.batch = tile / per_batch;
    tile -= t.batch * per_batch;
    constexpr int GM = 8;
    const int group = tile / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gm = min(p.tiles_m - first_m, GM);
    const int in_group = tile - group * GM * p.tiles_n;
    t.tm = first_m + in_group % gm;
    t.tn = in_group / gm;
    return t;
}

template <int BM, int BN, int BK, int WGM, int WGN, bool ALIGNED>
__global__ void __launch_bounds__(WGM* WGN * 64)
gemm_f16_mfma(GemmParams p) {
    constexpr int NT = WGM * WGN * 64;
    constexpr int WTM = BM / WGM;  // wave tile rows (m)
    constexpr int WTN = BN / WGN;  // wave tile cols (n)
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    constexpr int LDK = BK + 8;  // padded LDS row (halves): 16 B pad keeps b128 reads conflict-free
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && BK % 16 == 0, "tile shape");
    // A: 16-byte chunks
    constexpr int A_CHUNKS = BM * BK / 8;
    static_assert(A_CHUNKS % NT == 0, "A tile must split evenly over threads");
    constexpr int LA = A_CHUNKS / NT;
    // B: KR x 8 blocks (KR rows of K, 8 columns of N), transposed in registers
    constexpr int KR = (((BK / 8) * (BN / 8)) % NT == 0) ? 8 : 4;
    constexpr int B_BLOCKS = (BK / KR) * (BN / 8);
    static_assert(B_BLOCKS % NT == 0, "B tile must split evenly over threads");
    constexpr int LB = B_BLOCKS / NT;

    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];
    __shared__ int s_last;

    const TileCoord tc = decode_tile(p);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN;
    const int wn = wave % WGN;
    const int m0 = tc.tm * BM;
    const int n0 = tc.tn * BN;
    const int kbeg = tc.split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int ktiles = kend > kbeg ? cdiv(kend - kbeg, BK) : 0;

    const uint16_t* __restrict__ A = p.A + tc.batch * p.strideA;
    const uint16_t* __restrict__ B = p.B + tc.batch * p.strideB;
    uint16_t* __restrict__ C = p.C + tc.batch * p.strideC;
    const int M = p.M, N = p.N, K = p.K;

    unsigned ra[LA][4];
    unsigned rb[LB][KR][4];

    auto load_tiles = [&](int kt) {
        const int k0 = kbeg + kt * BK;
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int c = tid + i * NT;
            const int row = c / (BK / 8);
            const int kc = (c % (BK / 8)) * 8;
            const int gm = m0 + row;
            const int gk = k0 + kc;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (gm < M && gk < kend)
                    v = *reinterpret_cast<const u32x4*>(A + (int64_t)gm * K + gk);
                ra[i][0] = v.x; ra[i][1] = v.y; ra[i][2] = v.z; ra[i][3] = v.w;
            } else {
                uint16_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    h[e] = (gm < M && gk + e < kend) ? A[(int64_t)gm * K + gk + e] : (uint16_t)0;
#pragma unroll
                for (int d = 0; d < 4; ++d) ra[i][d] = h[2 * d] | ((unsigned)h[2 * d + 1] << 16);
            }
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = tid + i * NT;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
            const int gn = n0 + nb * 8;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                const int gk = k0 + kb * KR + r;
                if constexpr (ALIGNED) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (gk < kend && gn < N)
                        v = *reinterpret_cast<const u32x4*>(B + (int64_t)gk * N + gn);
                    rb[i][r][0] = v.x; rb[i][r][1] = v.y; rb[i][r][2] = v.z; rb[i][r][3] = v.w;
                } else {
                    uint16_t h[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        h[e] = (gk < kend && gn + e < N) ? B[(int64_t)gk * N + gn + e] : (uint16_t)0;
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        rb[i][r][d] = h[2 * d] | ((unsigned)h[2 * d + 1] << 16);
                }
            }
        }
    };

    auto store_tiles = [&](int st) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int c = tid + i * NT;
            const int row = c / (BK / 8);
            const int kc = (c % (BK / 8)) * 8;
            u32x4 v = {ra[i][0], ra[i][1], ra[i][2], ra[i][3]};
            *reinterpret_cast<u32x4*>(&sA[st][row * LDK + kc]) = v;
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int b = tid + i * NT;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                unsigned w[KR / 2];
#pragma unroll
                for (int j = 0; j < KR / 2; ++j) {
                    const unsigned lo = rb[i][2 * j][c >> 1];
                    const unsigned hi = rb[i][2 * j + 1][c >> 1];
                    w[j] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u))
                                   : ((lo & 0xffffu) | (hi << 16));
                }
                uint16_t* dst = &sB[st][(nb * 8 + c) * LDK + kb * KR];
                if constexpr (KR == 8) {
                    u32x4 v = {w[0], w[1], w[2], w[3]};
                    *reinterpret_cast<u32x4*>(dst) = v;
                } else {
                    u32x2 v = {w[0], w[1]};
                    *reinterpret_cast<u32x2*>(dst) = v;
                }
            }
        }
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (ktiles > 0) {
        load_tiles(0);
        store_tiles(0);
        __syncthreads();
    }
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 8;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load_tiles(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            f16x8 bf[FN], af[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i)
                bf[i] = lds_read_f16x8(&sB[st][(wn * WTN + i * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int j = 0; j < FM; ++j)
                af[j] = lds_read_f16x8(&sA[st][(wm * WTM + j * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_tiles(st ^ 1);
        __syncthreads();
    }

    // ---- split-K: publish partials, last arriver reduces in split order ----
    if (p.nsplit > 1) {
        const int tile_id = (tc.batch * p.tiles_m + tc.tm) * p.tiles_n + tc.tn;
        float* ws_tile = p.ws + (int64_t)tile_id * p.nsplit * (BM * BN);
        f32x4* mine = reinterpret_cast<f32x4*>(ws_tile + (int64_t)tc.split * (BM * BN));
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int v = (i * FM + j) * 4 + q;
                    f32x4 val = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                 acc[i][j][4 * q + 3]};
                    mine[v * NT + tid] = val;
                }
        if (!splitk_arrive_is_last(&p.counters[tile_id], (unsigned)p.nsplit, &s_last)) return;
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        for (int s = 0; s < p.nsplit; ++s) {
            const f32x4* part = reinterpret_cast<const f32x4*>(ws_tile + (int64_t)s * (BM * BN));
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 v = __builtin_nontemporal_load(&part[((i * FM + j) * 4 + q) * NT + tid]);
                        acc[i][j][4 * q] += v.x;
                        acc[i][j][4 * q + 1] += v.y;
                        acc[i][j][4 * q + 2] += v.z;
                        acc[i][j][4 * q + 3] += v.w;
                    }
        }
    }

    // ---- epilogue: lane holds C[m][n..n+3] for each (i, j, q) ----
    const float alpha = p.alpha, beta = p.beta;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int gm = m0 + wm * WTM + j * 32 + lrow;
            if (gm >= M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int gn = n0 + wn * WTN + i * 32 + q * 8 + (lane >> 5) * 4;
                float r[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) r[e] = alpha * acc[i][j][4 * q + e];
                uint16_t* dst = C + (int64_t)gm * N + gn;
                if constexpr (ALIGNED) {
                    if (gn >= N) continue;
                    if (beta != 0.0f) {
                        const u32x2 c = *reinterpret_cast<const u32x2*>(dst);
                        r[0] = fmaf(beta, h2f(c.x & 0xffffu), r[0]);
                        r[1] = fmaf(beta, h2f(c.x >> 16), r[1]);
                        r[2] = fmaf(beta, h2f(c.y & 0xffffu), r[2]);
                        r[3] = fmaf(beta, h2f(c.y >> 16), r[3]);
                    }
                    u32x2 o = {pack2h(r[0], r[1]), pack2h(r[2], r[3])};
                    *reinterpret_cast<u32x2*>(dst) = o;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (gn + e < N) {
                            float v = r[e];
                            if (beta != 0.0f) v = fmaf(beta, h2f(dst[e]), v);
                            dst[e] = f2h(v);
                        }
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV path for M <= 4 (decode).  Workgroup = 256 threads = 32 column lanes x
// 8 K lanes; each column lane owns 8 consecutive columns (one 16 B load per K
// row), so one wave covers 2 K rows x 256 columns (2 x 512 B contiguous).
// ---------------------------------------------------------------------------
struct GemvParams {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    int M, N, K;
    float alpha, beta;
    int64_t strideA, strideB, strideC;
    int col_blocks;   // cdiv(N, 256)
    int nsplit;
    int k_per_split;  // multiple of 8
    float* ws;
    unsigned* counters;
};

constexpr int GV_COLS = 256;
constexpr int GV_KL = 8;      // K lanes per workgroup
constexpr int GV_UNROLL = 8;  // B rows in flight per thread

template <int MM>
__global__ void __launch_bounds__(256) gemv_f16(GemvParams p) {
    __shared__ float red[GV_KL][MM][GV_COLS];
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int cl = tid & 31;
    const int kl = tid >> 5;
    int bid = blockIdx.x;
    const int split = bid % p.nsplit;
    bid /= p.nsplit;
    const int batch = bid / p.col_blocks;
    const int cb = bid - batch * p.col_blocks;
    const uint16_t* __restrict__ A = p.A + batch * p.strideA;
    const uint16_t* __restrict__ B = p.B + batch * p.strideB;
    uint16_t* __restrict__ C = p.C + batch * p.strideC;
    const int M = p.M, N = p.N, K = p.K;
    const int n = cb * GV_COLS + cl * 8;
    const bool col_ok = n < N;
    const int kbeg = split * p.k_per_split;
    const int kend = min(K, kbeg + p.k_per_split);

    float acc[MM][8];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;

    for (int k = kbeg + kl; k < kend; k += GV_KL * GV_UNROLL) {
        u32x4 bv[GV_UNROLL];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kk = k + u * GV_KL;
            bv[u] = (col_ok && kk < kend)
                        ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(B + (int64_t)kk * N + n))
                        : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kk = k + u * GV_KL;
            if (kk >= kend) break;
            float bf[8];
            bf[0] = h2f(bv[u].x & 0xffffu); bf[1] = h2f(bv[u].x >> 16);
            bf[2] = h2f(bv[u].y & 0xffffu); bf[3] = h2f(bv[u].y >> 16);
            bf[4] = h2f(bv[u].z & 0xffffu); bf[5] = h2f(bv[u].z >> 16);
            bf[6] = h2f(bv[u].w & 0xffffu); bf[7] = h2f(bv[u].w >> 16);
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const float a = (m < M) ? h2f(A[(int64_t)m * K + kk]) : 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[m][e] = fmaf(a, bf[e], acc[m][e]);
            }
        }
    }

    // reduce the 8 K lanes (fixed order)
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[kl][m][cl * 8 + e] = acc[m][e];
    __syncthreads();
    // thread t now owns column t of the block for every row
    const int col = tid;
    const int gn = cb * GV_COLS + col;
    float sum[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < GV_KL; ++q) s += red[q][m][col];
        sum[m] = s;
    }

    if (p.nsplit > 1) {
        const int tile_id = batch * p.col_blocks + cb;
        float* ws_tile = p.ws + (int64_t)tile_id * p.nsplit * (MM * GV_COLS);
#pragma unroll
        for (int m = 0; m < MM; ++m) ws_tile[(int64_t)split * MM * GV_COLS + m * GV_COLS + col] = sum[m];
        if (!splitk_arrive_is_last(&p.counters[tile_id], (unsigned)p.nsplit, &s_last)) return;
#pragma unroll
        for (int m = 0; m < MM; ++m) sum[m] = 0.0f;
        for (int s = 0; s < p.nsplit; ++s)
#pragma unroll
            for (int m = 0; m < MM; ++m)
                sum[m] += __builtin_nontemporal_load(&ws_tile[(int64_t)s * MM * GV_COLS + m * GV_COLS + col]);
    }
    if (gn < N) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (m < M) {
                float r = p.alpha * sum[m];
                uint16_t* dst = C + (int64_t)m * N + gn;
                if (p.beta != 0.0f) r = fmaf(p.beta, h2f(*dst), r);
                *dst = f2h(r);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
namespace {

struct SplitPlan {
    int nsplit;
    int k_per_split;
};

// Enough workgroups to cover every CU about twice, with at least `min_tiles`
// K tiles per split.
SplitPlan plan_split(int tiles, int K, int bk, int num_cus, int min_tiles) {
    SplitPlan sp{1, cdiv(K > 0 ? K : 1, bk) * bk};
    const int target = 2 * num_cus;
    if (tiles >= num_cus || K <= 0) return sp;
    const int ktiles = cdiv(K, bk);
    int want = cdiv(target, tiles);
    int maxs = max(1, ktiles / min_tiles);
    int ns = min(want, maxs);
    if (ns <= 1) return sp;
    const int kps = cdiv(ktiles, ns) * bk;
    sp.nsplit = cdiv(K, kps);
    sp.k_per_split = kps;
    return sp;
}

template <int BM, int BN, int BK, int WGM, int WGN, bool ALIGNED>
clove_status_t run_mfma(GemmParams p, int batch, int num_cus, hipStream_t stream) {
    p.tiles_m = cdiv(p.M, BM);
    p.tiles_n = cdiv(p.N, BN);
    const int tiles = p.tiles_m * p.tiles_n * batch;
    const SplitPlan sp = plan_split(tiles, p.K, BK, num_cus, 4);
    p.nsplit = sp.nsplit;
    p.k_per_split = sp.k_per_split;
    p.ws = nullptr;
    p.counters = nullptr;
    if (p.nsplit > 1) {
        Scratch s;
        const size_t bytes = (size_t)tiles * p.nsplit * BM * BN * sizeof(float);
        clove_status_t st = acquire_scratch(stream, bytes, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
    }
    const int64_t grid = (int64_t)tiles * p.nsplit;
    if (grid > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    hipLaunchKernelGGL((gemm_f16_mfma<BM, BN, BK, WGM, WGN, ALIGNED>), dim3((unsigned)grid),
                       dim3(WGM * WGN * 64), 0, stream, p);
    return check_launch();
}

template <int MM>
clove_status_t run_gemv(GemvParams p, int batch, int num_cus, hipStream_t stream) {
    p.col_blocks = cdiv(p.N, GV_COLS);
    const int tiles = p.col_blocks * batch;
    // split K so that ~4 workgroups run per CU; each split keeps >= 64 rows
    int want = cdiv(4 * num_cus, tiles);
    int maxs = max(1, p.K / 64);
    int ns = max(1, min(want, maxs));
    int kps = cdiv(cdiv(p.K, ns), 8) * 8;
    p.nsplit = cdiv(p.K, kps);
    p.k_per_split = kps;
    p.ws = nullptr;
    p.counters = nullptr;
    if (p.nsplit > 1) {
        Scratch s;
        const size_t bytes = (size_t)tiles * p.nsplit * MM * GV_COLS * sizeof(float);
        clove_status_t st = acquire_scratch(stream, bytes, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
    }
    hipLaunchKernelGGL((gemv_f16<MM>), dim3(tiles * p.nsplit), dim3(256), 0, stream, p);
    return check_launch();
}

}  // namespace
}  // namespace fp16

clove_status_t launch_gemm_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C, int batch,
                                int M, int N, int K, float alpha, float beta,
                                hipStream_t stream) {
    using namespace fp16;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const bool aligned = aligned16(A) && aligned16(B) && aligned16(C) && (K % 8 == 0) &&
                         (N % 8 == 0);
    const int64_t sA = (int64_t)M * K, sB = (int64_t)K * N, sC = (int64_t)M * N;

    if (aligned && M <= 4 && K > 0) {
        GemvParams g{A, B, C, M, N, K, alpha, beta, sA, sB, sC, 0, 1, 0, nullptr, nullptr};
        if (M == 1) return run_gemv<1>(g, batch, dev.num_cus, stream);
        if (M == 2) return run_gemv<2>(g, batch, dev.num_cus, stream);
        return run_gemv<4>(g, batch, dev.num_cus, stream);
    }
    GemmParams p{A, B, C, M, N, K, alpha, beta, sA, sB, sC, 0, 0, 1, 0, nullptr, nullptr};
    const int64_t big_tiles = (int64_t)cdiv(M, 256) * cdiv(N, 256) * batch;
    if (aligned) {
        if (big_tiles >= dev.num_cus / 2) return run_mfma<256, 256, 64, 2, 2, true>(p, batch, dev.num_cus, stream);
        if (M <= 32) return run_mfma<32, 128, 64, 1, 4, true>(p, batch, dev.num_cus, stream);
        if (M <= 64) return run_mfma<64, 128, 64, 2, 2, true>(p, batch, dev.num_cus, stream);
        return run_mfma<128, 128, 64, 2, 2, true>(p, batch, dev.num_cus, stream);
    }
    if (M <= 32) return run_mfma<32, 128, 64, 1, 4, false>(p, batch, dev.num_cus, stream);
    return run_mfma<128, 128, 64, 2, 2, false>(p, batch, dev.num_cus, stream);
}

}  // namespace clove
