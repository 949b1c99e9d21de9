// FP16 GEMM for gfx950: C = alpha * A @ B + beta * C, fp32 accumulation.
//
// Replaces the reference's gemm_fp16 (src/kernels/gemm_fp16.cu:277-305) and
// gemm_fp16_batched (:366-383).  Kernels:
//
//  * dma::gemm_f16_big (f16_dma_gemm.hpp) -- large aligned shapes: 256x256x64
//    tiles of v_mfma_f32_16x16x32_f16, A and B staged by LDS DMA, B fragments
//    from transposing LDS reads, one tile per CU.
//  * mg::mfma_gemm with the fp16 row loader for A and the transposing fp16
//    column loader for B (mfma_gemm.hpp): LDS-tiled v_mfma_f32_32x32x16_f16,
//    tile shape chosen per (M, N), split-K when the tile grid is too small to
//    fill the CUs; every other shape.
//  * gemv_f16 -- M <= 4 decode shapes: B streamed once from HBM with 16 B
//    loads (a 256 x 256 tile per workgroup, all in flight), fp32 FMAs on the
//    VALU, split-K over workgroups.
#include "common.hpp"
#include "dispatch.hpp"
#include "f16_dma_gemm.hpp"
#include "mfma_gemm.hpp"

namespace clove {
namespace fp16 {

using namespace hw;

// ---------------------------------------------------------------------------
// GEMV path for M <= 4 (decode).  A workgroup of 1024 threads owns 256
// columns x 256 k-rows of B: thread (kl, cl) = (tid / 32, tid % 32) loads the
// 16 bytes of columns 8cl..8cl+7 of rows kl + 32j, j < 8, so each wave
// instruction reads two full 512-byte row segments and the whole 128 KB tile is
// requested at once.  Loads are unconditional from clamped addresses (masked
// at use).  Partials: wave halves (v_permlane32_swap), then the 16 waves
// through LDS (fixed order), then the K splits, summed by the last workgroup
// to arrive (coherent stores and loads, split order).
// ---------------------------------------------------------------------------
struct GemvParams {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    const uint16_t* B2;  // SWIGLU: the up projection's weights (B holds the gate's)
    int M, N, K;
    float alpha, beta;
    int64_t strideA, strideB, strideC;
    int col_blocks;   // cdiv(N, 256)
    int nsplit;       // cdiv(K, 256)
    float* ws;
    unsigned* counters;
};

constexpr int GV_COLS = 256;
constexpr int GV_KL = 32;                 // k lanes
constexpr int GV_RPT = 8;                 // rows per thread
constexpr int GV_ROWS = GV_KL * GV_RPT;   // k rows per workgroup

// SWIGLU: the workgroup's 256 columns are 128 columns of B (gate) and the
// same 128 columns of B2 (up): column lanes 0..15 read B, 16..31 read B2, so a
// wave instruction reads two 256-byte row segments.  Every column's sum runs
// over the same k in the same order as in the one-operand kernel (the k
// mapping does not depend on the column), so gate and up are bit-identical
// to two gemm_fp16 calls; the epilogue rounds both to fp16 and applies SwiGLU.
template <int MM, bool SWIGLU = false>
__global__ void __launch_bounds__(1024) gemv_f16(GemvParams p) {
    __shared__ float red[16][MM][GV_COLS];
    __shared__ float s_up[SWIGLU ? MM : 1][SWIGLU ? GV_COLS / 2 : 1];
    __shared__ int s_last;
    constexpr int CW = SWIGLU ? GV_COLS / 2 : GV_COLS;  // output columns per workgroup
    const int tid = threadIdx.x;
    const int cl = tid & 31, kl = tid >> 5, wave = tid >> 6;
    int bid = blockIdx.x;
    const int split = bid % p.nsplit;
    bid /= p.nsplit;
    const int batch = bid / p.col_blocks;
    const int cb = bid - batch * p.col_blocks;
    const uint16_t* __restrict__ A = p.A + batch * p.strideA;
    const uint16_t* __restrict__ B = (SWIGLU && cl >= 16 ? p.B2 : p.B) + batch * p.strideB;
    uint16_t* __restrict__ C = p.C + batch * p.strideC;
    const int M = p.M, N = p.N, K = p.K;
    const int n = cb * CW + (SWIGLU ? cl & 15 : cl) * 8;
    const int nc = min(n, N - 8);
    const int kbeg = split * GV_ROWS;

    // A (small, shared by every workgroup) first: loads complete in order, so
    // the FMAs of row j wait only for B row j, not for the whole tile
    uint16_t xa[MM][GV_RPT];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int j = 0; j < GV_RPT; ++j)
            xa[m][j] = A[(int64_t)min(m, M - 1) * K + min(kbeg + kl + GV_KL * j, K - 1)];
    // (kept ahead of the B loads: one A load scheduled after them would make
    // the first FMA wait for every B row, loads completing in order)
    __builtin_amdgcn_sched_barrier(0);
    u32x4 bv[GV_RPT];
#pragma unroll
    for (int j = 0; j < GV_RPT; ++j) {
        const int k = min(kbeg + kl + GV_KL * j, K - 1);
        bv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(B + (int64_t)k * N + nc));
    }
    __builtin_amdgcn_sched_barrier(0);  // every B row requested before the first FMA

    float acc[MM][8];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;
#pragma unroll
    for (int j = 0; j < GV_RPT; ++j) {
        const bool row_ok = kbeg + kl + GV_KL * j < K;
        float bf[8];
        bf[0] = h2f(bv[j].x & 0xffffu); bf[1] = h2f(bv[j].x >> 16);
        bf[2] = h2f(bv[j].y & 0xffffu); bf[3] = h2f(bv[j].y >> 16);
        bf[4] = h2f(bv[j].z & 0xffffu); bf[5] = h2f(bv[j].z >> 16);
        bf[6] = h2f(bv[j].w & 0xffffu); bf[7] = h2f(bv[j].w >> 16);
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float a = (row_ok && m < M) ? h2f(xa[m][j]) : 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[m][e] = fmaf(a, bf[e], acc[m][e]);
        }
    }
    // the two k lanes of a wave (lanes l and l + 32, summed in that order) by
    // a half-wave swap: lanes 0..31 keep the even columns of their 8, lanes
    // 32..63 the odd ones; then the 16 waves through LDS
    const int half = (tid >> 5) & 1;
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int e = 0; e < 8; e += 2) red[wave][m][cl * 8 + e + half] = halves_sum2(acc[m][e], acc[m][e + 1]);
    __syncthreads();
    // threads 0..255 own one column each from here on; every thread still
    // takes part in the arrival barrier
    const bool active = tid < GV_COLS;
    const int col = active ? tid : 0;
    const int gn = cb * GV_COLS + col;
    float sum[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) s += red[w][m][col];
        sum[m] = s;
    }

    if (p.nsplit > 1) {
        const int tile_id = batch * p.col_blocks + cb;
        float* ws_tile = p.ws + (int64_t)tile_id * p.nsplit * (MM * GV_COLS);
        if (active) {
#pragma unroll
            for (int m = 0; m < MM; ++m)
                store_coherent(&ws_tile[(int64_t)split * MM * GV_COLS + m * GV_COLS + col], sum[m]);
        }
        if (!splitk_arrive_is_last(&p.counters[tile_id], (unsigned)p.nsplit, &s_last)) return;
#pragma unroll
        for (int m = 0; m < MM; ++m) sum[m] = 0.0f;
        // all partials in flight at once (none past the last split), then
        // summed in split order
        for (int s0 = 0; s0 < p.nsplit; s0 += 16) {
            float part[16][MM];
#pragma unroll
            for (int s = 0; s < 16; ++s)
#pragma unroll
                for (int m = 0; m < MM; ++m)
                    part[s][m] = s0 + s < p.nsplit
                                     ? load_coherent(&ws_tile[(int64_t)(s0 + s) * MM * GV_COLS + m * GV_COLS + col])
                                     : 0.0f;
#pragma unroll
            for (int s = 0; s < 16; ++s)
#pragma unroll
                for (int m = 0; m < MM; ++m) sum[m] += part[s][m];
        }
    }
    if constexpr (SWIGLU) {
        // columns 128..255 of the workgroup are the up sums of columns 0..127
        if (active && tid >= CW) {
#pragma unroll
            for (int m = 0; m < MM; ++m) s_up[m][tid - CW] = sum[m];
        }
        __syncthreads();
        if (tid >= CW) return;
        const int go = cb * CW + tid;
        if (go < N) {
#pragma unroll
            for (int m = 0; m < MM; ++m)
                if (m < M) C[(int64_t)m * N + go] = swiglu_h(f2h(sum[m]), f2h(s_up[m][tid]));
        }
        return;
    }
    if (!active) return;
    if (gn < N) {
        // beta != 0: the old outputs are loaded (clamped rows) before the first store
        float old[MM];
        if (p.beta != 0.0f) {
#pragma unroll
            for (int m = 0; m < MM; ++m) old[m] = h2f(C[(int64_t)min(m, M - 1) * N + gn]);
        }
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (m < M) {
                float r = p.alpha * sum[m];
                if (p.beta != 0.0f) r = fmaf(p.beta, old[m], r);
                C[(int64_t)m * N + gn] = f2h(r);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
namespace {

using mg::Params;
using mg::Tile;

template <class T, bool ALIGNED>
clove_status_t run_mfma(Params p, int batch, int num_cus, hipStream_t stream) {
    using LA = mg::LoadF16Rows<T::BM, T::BK, T::NT, T::LDK, false, ALIGNED>;
    using LB = mg::LoadF16Cols<T::BN, T::BK, T::NT, T::LDK, ALIGNED>;
    p.tiles_m = cdiv(p.M, T::BM);
    p.tiles_n = cdiv(p.N, T::BN);
    const int tiles = p.tiles_m * p.tiles_n * batch;
    const mg::SplitPlan sp = mg::plan_split(tiles, p.K, T::BK, num_cus, 2 * num_cus, 4);
    p.nsplit = sp.nsplit;
    p.k_per_split = sp.k_per_split;
    p.ws = nullptr;
    p.counters = nullptr;
    if (p.nsplit > 1) {
        Scratch s;
        const size_t bytes = (size_t)tiles * p.nsplit * T::BM * T::BN * sizeof(float);
        clove_status_t st = acquire_scratch(stream, bytes, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
    }
    const int64_t grid = (int64_t)tiles * p.nsplit;
    if (grid > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    if (p.nsplit > 1)
        CLOVE_LAUNCH((mg::mfma_gemm<T, LA, LB, mg::EpiAlphaBeta<ALIGNED>, mg::kFoldNone, true>),
                           dim3((unsigned)grid), dim3(T::NT), 0, stream, p);
    else
        CLOVE_LAUNCH((mg::mfma_gemm<T, LA, LB, mg::EpiAlphaBeta<ALIGNED>, mg::kFoldNone, false>),
                           dim3((unsigned)grid), dim3(T::NT), 0, stream, p);
    return check_launch();
}

using BigTile = dma::Big;

// The DMA kernel's preconditions: 16-byte aligned operands, K a multiple of
// the K tile, N a multiple of 8, every per-batch operand addressable with
// 32-bit byte offsets.
bool dma_eligible(const void* A, const void* B, const void* C, int M, int N, int K) {
    return aligned16(A) && aligned16(B) && aligned16(C) && K > 0 && K % BigTile::BK == 0 &&
           N % 8 == 0 && N >= 8 && M >= 1 && (int64_t)M * K * 2 < (1ll << 31) &&
           (int64_t)K * N * 2 < (1ll << 31) && (int64_t)M * N * 2 < (1ll << 31);
}

// The K split of the 256x256 kernel.  When its tiles cover only half the CUs
// (the kernel is chosen from cus / 2 tiles up; M x N = 128 tiles of 256 x 256
// on this part, e.g. 2048 x 4096) and K is long, each tile's K range is split
// in two: every CU runs a half-length tile, both halves publish fp32 partial
// tiles (256 KB each) and the last to arrive sums them in split order.
// Measured against the same 128 tiles unsplit: K = 11008 164-169 against
// 207-210 us; K = 4096 82-84 against 84-102 (half the chip idle runs at a
// higher clock), so only from K = 8192.  Not above cus / 2 tiles: splitting
// the remainder of a partly filled last round (2048 x 11008 x 4096, 344 tiles)
// measured no faster (185.6 against 187.8 us), the partials' traffic (1 MB per
// split tile) costing what the shorter round saved.
struct BigSplit {
    int nsplit = 1, ktps = 0;
};
BigSplit big_split_plan(int64_t tiles, int batch, int KT, int cus) {
    BigSplit sp;
    if (batch != 1 || 2 * tiles > cus || KT < 128) return sp;
    sp.ktps = cdiv(KT, 2);
    sp.nsplit = cdiv(KT, sp.ktps);
    return sp;
}

clove_status_t run_dma(const uint16_t* A, const uint16_t* B, uint16_t* C, int batch, int M, int N,
                       int K, float alpha, float beta, int cus, hipStream_t stream) {
    dma::Args a{A, B, C, M, N, K, alpha, beta, (int64_t)M * K, (int64_t)K * N, (int64_t)M * N,
                cdiv(M, BigTile::BM), cdiv(N, BigTile::BN)};
    const int64_t grid = (int64_t)a.tiles_m * a.tiles_n * batch;
    if (grid > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    const BigSplit sp = big_split_plan(grid, batch, K / BigTile::BK, cus);
    if (sp.nsplit > 1) {
        constexpr size_t kSlab = (size_t)BigTile::FM * BigTile::FN * BigTile::NT * 16;  // one part's tile
        Scratch s;
        const clove_status_t st = acquire_scratch(stream, (size_t)grid * sp.nsplit * kSlab, (size_t)grid, &s);
        if (st != CLOVE_OK) return st;
        a.nsplit = sp.nsplit;
        a.ktps = sp.ktps;
        a.part = s.partials;
        a.counters = s.counters;
        CLOVE_LAUNCH(dma::gemm_f16_big_split<dma::Big>, dim3((unsigned)(grid * sp.nsplit)), dim3(BigTile::NT), 0,
                     stream, a);
        return check_launch();
    }
    CLOVE_LAUNCH(dma::gemm_f16_big<dma::Big>, dim3((unsigned)grid), dim3(BigTile::NT), 0, stream, a);
    return check_launch();
}

template <int MM, bool SWIGLU = false>
clove_status_t run_gemv(GemvParams p, int batch, hipStream_t stream) {
    p.col_blocks = cdiv(p.N, SWIGLU ? GV_COLS / 2 : GV_COLS);
    p.nsplit = cdiv(p.K, GV_ROWS);
    const int tiles = p.col_blocks * batch;
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
    const int64_t grid = (int64_t)tiles * p.nsplit;
    if (grid > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    CLOVE_LAUNCH((gemv_f16<MM, SWIGLU>), dim3((unsigned)grid), dim3(1024), 0, stream, p);
    return check_launch();
}

}  // namespace
}  // namespace fp16

bool try_gemv_swiglu(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up, uint16_t* out, int T,
                     int hidden, int inter, hipStream_t stream, clove_status_t* status) {
    using namespace fp16;
    if (T < 1 || T > 4 || hidden <= 0 || hidden % 8 != 0 || inter < 8 || inter % 8 != 0) return false;
    if (!aligned16(X) || !aligned16(W_gate) || !aligned16(W_up) || !aligned16(out)) return false;
    const int64_t sA = (int64_t)T * hidden, sB = (int64_t)hidden * inter, sC = (int64_t)T * inter;
    GemvParams g{X, W_gate, out, W_up, T, inter, hidden, 1.0f, 0.0f, sA, sB, sC, 0, 1, nullptr, nullptr};
    if (T == 1) *status = run_gemv<1, true>(g, 1, stream);
    else if (T == 2) *status = run_gemv<2, true>(g, 1, stream);
    else *status = run_gemv<4, true>(g, 1, stream);
    return true;
}

bool fp16_takes_big_tile(const void* A, const void* B, const void* C, int M, int N, int K, int cus) {
    using namespace fp16;
    return M > 4 && (int64_t)cdiv(M, 256) * cdiv(N, 256) >= cus / 2 && dma_eligible(A, B, C, M, N, K);
}

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

    if (skinny_before_gemv(M, N, K)) {
        clove_status_t st2;
        if (try_skinny_fp16(A, B, C, batch, M, N, K, alpha, beta, dev.num_cus, stream, &st2)) return st2;
    }
    if (aligned && M <= 4 && K > 0) {
        GemvParams g{A, B, C, nullptr, M, N, K, alpha, beta, sA, sB, sC, 0, 1, nullptr, nullptr};
        if (M == 1) return run_gemv<1>(g, batch, stream);
        if (M == 2) return run_gemv<2>(g, batch, stream);
        return run_gemv<4>(g, batch, stream);
    }
    Params p{};
    p.a = A; p.b = B; p.c = C;
    p.M = M; p.N = N; p.K = K;
    p.alpha = alpha; p.beta = beta;
    p.strideA = sA; p.strideB = sB; p.strideC = sC;
    const int cus = dev.num_cus;
    const int64_t big_tiles = (int64_t)cdiv(M, 256) * cdiv(N, 256) * batch;
    if (big_tiles >= cus / 2 && dma_eligible(A, B, C, M, N, K))
        return run_dma(A, B, C, batch, M, N, K, alpha, beta, cus, stream);
    {
        clove_status_t st2;
        if (try_skinny_fp16(A, B, C, batch, M, N, K, alpha, beta, cus, stream, &st2)) return st2;
    }
    if (aligned) {
        if (M <= 32) return run_mfma<Tile<32, 128, 64, 1, 4>, true>(p, batch, cus, stream);
        if (M <= 64) return run_mfma<Tile<64, 128, 64, 2, 2>, true>(p, batch, cus, stream);
        if (M <= 192) return run_mfma<Tile<128, 64, 128, 2, 2>, true>(p, batch, cus, stream);
        return run_mfma<Tile<128, 128, 64, 2, 2>, true>(p, batch, cus, stream);
    }
    if (M <= 32) return run_mfma<Tile<32, 128, 64, 1, 4>, false>(p, batch, cus, stream);
    return run_mfma<Tile<128, 128, 64, 2, 2>, false>(p, batch, cus, stream);
}

}  // namespace clove
