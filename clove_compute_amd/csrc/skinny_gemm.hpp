// GEMM for few rows of A (M <= 128) against a large N-contiguous B on gfx950:
// the prefill/small-batch shapes of gemm_fp16 and gemm_int8, where the run
// time is streaming B (the weights) from HBM once.
//
//   acc[m, n] = sum_k A[m, k] * B[k, n]      fp16 -> fp32, or int8 -> int32
//
// Both operands go global -> LDS by LDS DMA (buffer_load_dwordx4 ... lds, no
// VGPR staging), several stages in flight.  B stays N-contiguous in LDS and
// its MFMA fragments come from the transposing LDS reads: within a 16-lane
// group, ds_read_b64_tr_b16 gives result lane j element r = source lane
// (4 r + j / 4) element (j % 4), and ds_read_b64_tr_b8 gives result lane j
// byte r = source lane (2 r + j / 8) byte (j % 8); with source lane s of a
// group pointing at 8 bytes of k-row kb + s / 4 (fp16; s / 2 for int8),
// columns of the group's 16, every result lane receives 4 (8) consecutive k
// of one column.  Two such reads make the 16-byte MFMA operand.
//
// LDS layout per stage (16-byte chunks XOR-swizzled so that every fragment
// read is bank-conflict free):
//   A  BM rows x 128 bytes of k:   chunk c of row m at c ^ (m & 7)
//   B  BK k-rows x BNB bytes of n: chunk c of row r at c ^ swz_b(r)
// MFMA: v_mfma_f32_32x32x16_f16 / v_mfma_i32_32x32x32_i8 with the B fragment
// as the "A" operand (rows = n) and the A fragment as "B" (cols = m): a lane
// holds one row m and 4-column runs of n.  A k-step consumes 32 bytes of k.
//
// Split-K over workgroups (whole K tiles) when the tile grid does not cover
// the CUs, with the shared publish / reduce (split order, deterministic;
// int32 partials for INT8, so the integer accumulator stays exact).
//
// K slices (KW > 1, FP16 only, no split K): the small products (short K, a
// 32x32 tile per CU or fewer) run 32x32 tiles whose four waves each take one
// of every K tile's four k-steps; after the K loop every wave stores its sums
// to LDS and each wave adds the four slices, in slice order, for a quarter of
// the tile's output runs.
//
// Two B operands (NB = 2, FP16 only): B and B2 share A and the tile's
// columns; each stage holds A, then the B tile, then the B2 tile, and every
// wave keeps both accumulator sets.  The SwiGLU epilogue (kF16SwiGLU) then
// writes fp16(silu(fp16(A@B)) * fp16(A@B2)) -- gate and up of an MLP -- with
// neither projection reaching memory.  Each accumulator sums its k in the
// same order as the one-operand kernel with the same BM, BN and split plan,
// so gate and up are bit-identical to two separate GEMMs.
#pragma once

#include "common.hpp"
#include "f16_dma_gemm.hpp"

namespace clove {
namespace sk {

using namespace hw;
using dma::dma16;
using dma::make_rsrc;
using dma::vmcnt_imm;

enum Out { kF16AlphaBeta = 0, kI8Tensor = 1, kI8RowCol = 2, kI8Acc32 = 3, kF16SwiGLU = 4 };

struct Args {
    const void* A;       // [batch][M, K]
    const void* B;       // [batch][K, N]
    const void* B2;      // [batch][K, N], second B operand (NB = 2)
    void* C;             // [batch][M, N]  fp16, or int32 for kI8Acc32
    const uint16_t* sa;  // [M] fp16 (kI8RowCol)
    const uint16_t* sb;  // [N] fp16 (kI8RowCol)
    float scale;         // kI8Tensor
    float alpha, beta;   // kF16AlphaBeta
    int M, N, K;
    int64_t sA, sB, sC;  // batch strides, elements
    int tiles_m, tiles_n, batch, nsplit, kps;  // kps: K per split (multiple of BK)
    float* part;
    unsigned* counters;
};

// KW > 1: KW waves share each wave tile and take disjoint slices of every K
// tile's four k-steps, summed through LDS after the K loop (slice order, so
// deterministic): KW times the workgroups of the same wave tiles for small
// products (no split K)
template <bool I8_, int BM_, int BN_, int WM_, int WN_, int S_, int NB_ = 1, int KW_ = 1>
struct Cfg {
    static constexpr bool I8 = I8_;
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, S = S_, NB = NB_, KW = KW_;
    static constexpr int ES = I8 ? 1 : 2;  // bytes per element
    static constexpr int NW = WM * WN * KW, NT = 64 * NW;
    static constexpr int NKS = 4 / KW;     // k-steps per K tile per wave
    static constexpr int BK = 128 / ES;    // K per stage: 128 bytes of every A row
    static constexpr int BNB = BN * ES;    // bytes of one B k-row in the tile
    static constexpr int FM = BM / (32 * WM), FN = BN / (32 * WN);
    static constexpr int A_BYTES = BM * 128, B_BYTES = BK * BNB;
    static constexpr int SB = A_BYTES + NB * B_BYTES;
    static constexpr int DA = A_BYTES / 1024 / NW, DB = B_BYTES / 1024 / NW;  // DB per B operand
    static constexpr int D = DA + NB * DB;  // DMA instructions per thread per stage
    static_assert(NW == 4, "four waves");
    static_assert(NB == 1 || (NB == 2 && !I8), "two B operands: FP16 only");
    static_assert(FM >= 1 && FN >= 1 && BM == 32 * FM * WM && BN == 32 * FN * WN, "wave tiles");
    static_assert(BNB == 64 || BNB == 128 || BNB == 256 || BNB == 512, "B row bytes");
    static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "DMA split");
    static_assert(S >= 2 && S <= 9 && (S - 2) * D <= 63, "stages");
    static_assert(KW == 1 || ((KW == 2 || KW == 4) && !I8), "k slices");
    // the k-slice sums: every wave's NB FN FM 32x32 blocks, 4 KB each
    static constexpr int RED = KW > 1 ? NW * NB * FN * FM * 4096 : 0;
    static constexpr int LDS = S * SB + RED;
    static_assert(LDS <= 160 * 1024, "LDS");
};

// chunk swizzle of B k-row r (see the header comment): the rows one
// transposing read touches (4 rows x 2 chunks for fp16, 8 rows x 1 chunk for
// int8) land in 8 different bank groups
// (rows of 128 or 256 bytes start on bank 0, rows of 64 bytes alternate halves)
template <int BNB, bool I8>
__device__ __forceinline__ int swz_b(int r) {
    if constexpr (BNB >= 128) return I8 ? (r & 7) : 2 * (r & 3);
    else return I8 ? ((r >> 1) & 3) : 2 * ((r >> 1) & 1);
}

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef int i32x2v __attribute__((vector_size(8)));
typedef short i16x4v __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) i32x2v lds_i32x2v;
typedef __attribute__((address_space(3))) i16x4v lds_i16x4v;

__device__ __forceinline__ u32x4 lds_read16(unsigned a) { return *reinterpret_cast<const lds_u32x4*>((size_t)a); }

template <bool I8>
__device__ __forceinline__ u32x2 lds_read_tr(unsigned a) {
    if constexpr (I8) {
        const i32x2v v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_i32x2v*>((size_t)a));
        return u32x2{(unsigned)v[0], (unsigned)v[1]};
    } else {
        const i16x4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4v*>((size_t)a));
        return bitcast<u32x2>(v);
    }
}

// wait until stage t has landed, `ahead` later stages may stay in flight,
// then the workgroup barrier
// (ahead <= S - 2)
template <int S, int D, int A = S - 2>
__device__ __forceinline__ void stage_wait(int ahead) {
    if constexpr (A >= 1) {
        if (ahead >= A) {
            dma::stage_barrier<vmcnt_imm(A * D)>();
            return;
        }
        stage_wait<S, D, A - 1>(ahead);
    } else {
        dma::stage_barrier<vmcnt_imm(0)>();
    }
}

template <class CF, int OUT>
__global__ void __launch_bounds__(CF::NT) skinny_gemm(Args p) {
    constexpr int ES = CF::ES, NW = CF::NW, FM = CF::FM, FN = CF::FN, S = CF::S;
    constexpr int BM = CF::BM, BN = CF::BN, BK = CF::BK, BNB = CF::BNB, SB = CF::SB;
    constexpr int D = CF::D;
    constexpr bool I8 = CF::I8;
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave / (CF::WM * CF::WN);  // k slice (0 unless KW > 1)
    const int wmn = wave - kw * (CF::WM * CF::WN);
    const int wm = wmn % CF::WM, wn = wmn / CF::WM;
    constexpr int NKS = CF::NKS;

    // ---- tile, split, K range ----
    // Workgroups are dealt to the 8 XCDs round-robin (workgroup b runs on XCD
    // b % 8) and each XCD has its own L2: the grid is renumbered so that every
    // XCD owns a contiguous run of logical workgroups.  Logical order is
    // split-major (the workgroups in flight together share K rows of B), and
    // within a split the tiles are walked in groups of 8 tile-rows, column by
    // column, so one XCD's run shares a few A row panels and B column panels
    // instead of touching every A panel.
    int bid = blockIdx.x;
    if ((gridDim.x & 7) == 0) bid = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);
    const int ntiles = p.tiles_m * p.tiles_n * p.batch;
    const int split = bid / ntiles;
    int tile = bid - split * ntiles;
    const int per_batch = p.tiles_m * p.tiles_n;
    const int batch = tile / per_batch;
    const int t_in = tile - batch * per_batch;
    constexpr int GM = 8;
    const int group = t_in / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gm = min(p.tiles_m - first_m, GM);
    const int in_group = t_in - group * GM * p.tiles_n;
    const int tm = first_m + in_group % gm, tn = in_group / gm;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;
    const int kbeg = split * p.kps;
    const int nkt = (min(K, kbeg + p.kps) - kbeg) / BK;

    const unsigned lds0 = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) unsigned char*)smem));

    const unsigned char* Ab = static_cast<const unsigned char*>(p.A) + batch * p.sA * ES;
    const unsigned char* Bb = static_cast<const unsigned char*>(p.B) + batch * p.sB * ES;
    const u32x4 ra = make_rsrc(Ab, (unsigned)M * K * ES);
    const u32x4 rb = make_rsrc(Bb, (unsigned)K * N * ES);
    const u32x4 rb2 = CF::NB == 2
        ? make_rsrc(static_cast<const unsigned char*>(p.B2) + batch * p.sB * ES, (unsigned)K * N * ES)
        : rb;

    // ---- per-lane DMA offsets (fixed over K; the K position is the soffset) ----
    int offa[CF::DA], offb[CF::DB];
#pragma unroll
    for (int i = 0; i < CF::DA; ++i) {
        const int row = 8 * (wave * CF::DA + i) + (lane >> 3);
        offa[i] = (m0 + row) * K * ES + 16 * ((lane & 7) ^ (row & 7));
    }
    constexpr int CPR = BNB / 16, RPI = 1024 / BNB;  // chunks per B row, rows per instruction
#pragma unroll
    for (int i = 0; i < CF::DB; ++i) {
        const int row = RPI * (wave * CF::DB + i) + lane / CPR;
        offb[i] = row * N * ES + n0 * ES + 16 * ((lane % CPR) ^ swz_b<BNB, I8>(row));
    }
    auto issue = [&](int t, int stage) {
        const int k0 = kbeg + t * BK;
        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(stage * SB));
#pragma unroll
        for (int i = 0; i < CF::DA; ++i) dma16(ra, st + (wave * CF::DA + i) * 1024, offa[i], k0 * ES);
#pragma unroll
        for (int i = 0; i < CF::DB; ++i)
            dma16(rb, st + CF::A_BYTES + (wave * CF::DB + i) * 1024, offb[i], k0 * N * ES);
        if constexpr (CF::NB == 2) {
#pragma unroll
            for (int i = 0; i < CF::DB; ++i)
                dma16(rb2, st + CF::A_BYTES + CF::B_BYTES + (wave * CF::DB + i) * 1024, offb[i], k0 * N * ES);
        }
    };

    // ---- fragment addressing (relative to the stage) ----
    const int kh = lane >> 5, l32 = lane & 31;
    // A: row wm*32FM + 32j + l32, k-step t reads chunk (2t + kh) ^ (l & 7); tile j is +4096 j.
    // The wave's k-steps of a K tile are t = NKS kw + u, u < NKS.
    unsigned aoff[NKS];
#pragma unroll
    for (int u = 0; u < NKS; ++u) {
        const int t = NKS * kw + u;
        aoff[u] = (wm * 32 * FM + l32) * 128 + 16 * ((2 * t + kh) ^ (lane & 7));
    }
    // B: group g = l32 / 16 covers columns wn*32FN + 32i + 16g .. +15; source lane s = lane & 15
    // points at k-row (step rows) + s / RL and byte 8 (s % LR) of the group's columns
    constexpr int RL = I8 ? 2 : 4;        // lanes per k-row in one transposing read
    constexpr int RR = 16 / RL;           // k-rows per transposing read
    const int s16 = lane & 15, g = l32 >> 4;
    // (the swizzle mixes chunk bits that distinguish the tiles i, so every
    // tile has its own offsets)
    unsigned boff[NKS][2][FN];            // [k-step][read][tile]
#pragma unroll
    for (int u = 0; u < NKS; ++u)
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int t = NKS * kw + u;
                const int row = t * (32 / ES) + kh * (16 / ES) + e * RR + s16 / RL;
                const int col = (wn * 32 * FN + 32 * i + 16 * g) * ES + 8 * (s16 % RL);
                boff[u][e][i] = CF::A_BYTES + row * BNB + 16 * ((col >> 4) ^ swz_b<BNB, I8>(row)) + (col & 15);
            }

    typedef typename std::conditional<I8, i32x16, f32x16>::type AccT;
    typedef typename std::conditional<I8, i32x4, f32x4>::type AccT4;
    constexpr int NB = CF::NB;
    static_assert((OUT == kF16SwiGLU) == (NB == 2), "the SwiGLU epilogue takes two B operands");
    AccT acc[NB][FN][FM];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[b][i][j][v] = 0;

#pragma unroll
    for (int t = 0; t < S - 1; ++t)
        if (t < nkt) issue(t, t);

    int stage = 0, stage_next = S - 1;
    for (int t = 0; t < nkt; ++t) {
        stage_wait<S, D>(min(S - 2, nkt - 1 - t));
        if (t + S - 1 < nkt) issue(t + S - 1, stage_next);
        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(stage * SB));
        stage_next = stage;
        stage = stage + 1 == S ? 0 : stage + 1;

#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            u32x4 af[FM];
            const unsigned ab = st + aoff[ks];
#pragma unroll
            for (int j = 0; j < FM; ++j) af[j] = lds_read16(ab + 4096 * j);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                u32x4 bf[FN];
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    const u32x2 lo = lds_read_tr<I8>(st + b * CF::B_BYTES + boff[ks][0][i]);
                    const u32x2 hi = lds_read_tr<I8>(st + b * CF::B_BYTES + boff[ks][1][i]);
                    bf[i] = u32x4{lo.x, lo.y, hi.x, hi.y};
                }
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int j = 0; j < FM; ++j) {
                        if constexpr (I8)
                            acc[b][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                                bitcast<i32x4>(bf[i]), bitcast<i32x4>(af[j]), acc[b][i][j], 0, 0, 0);
                        else
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                bitcast<f16x8>(bf[i]), bitcast<f16x8>(af[j]), acc[b][i][j], 0, 0, 0);
                    }
            }
        }
    }

    // ---- k slices: every wave stores its sums to LDS; wave kw then owns the
    // runs q with q / (4 / KW) == kw of every block and adds the KW slices in
    // slice order ----
    constexpr int NQ = 4 / CF::KW;  // runs of 4 columns per block owned by a wave
    if constexpr (CF::KW > 1) {
        const unsigned red = lds0 + (unsigned)(S * SB);
        // wave tile wmn, slice s, block (b, i, j), run q: 1 KB, 16 lane-contiguous
        // bytes per lane
        auto slot = [&](int s, int b, int i, int j, int q) {
            return red +
                   (unsigned)(((((((wmn * CF::KW + s) * NB + b) * FN + i) * FM + j) * 4 + q) << 10) + 16 * lane);
        };
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<lds_u32x4*>((size_t)slot(kw, b, i, j, q)) = bitcast<u32x4>(
                            f32x4{acc[b][i][j][4 * q], acc[b][i][j][4 * q + 1], acc[b][i][j][4 * q + 2],
                                  acc[b][i][j][4 * q + 3]});
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (q / NQ != kw) continue;
                        f32x4 sum = bitcast<f32x4>(lds_read16(slot(0, b, i, j, q)));
#pragma unroll
                        for (int s = 1; s < CF::KW; ++s) {
                            const f32x4 v = bitcast<f32x4>(lds_read16(slot(s, b, i, j, q)));
                            sum = f32x4{sum[0] + v[0], sum[1] + v[1], sum[2] + v[2], sum[3] + v[3]};
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[b][i][j][4 * q + e] = sum[e];
                    }
    }

    // ---- split-K (not with k slices: the host plans none) ----
    if (CF::KW == 1 && p.nsplit > 1) {
        constexpr int NC = NB * FN * FM * 4;
        f32x4 v[NC];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        v[((b * FN + i) * FM + j) * 4 + q] = bitcast<f32x4>(
                            AccT4{acc[b][i][j][4 * q], acc[b][i][j][4 * q + 1], acc[b][i][j][4 * q + 2],
                                  acc[b][i][j][4 * q + 3]});
        float* slabs = p.part + (size_t)tile * p.nsplit * NC * CF::NT * 4;
        splitk_publish<NC, CF::NT>(slabs + (size_t)split * NC * CF::NT * 4, tid, v);
        if (!splitk_arrive_is_last(p.counters + tile, (unsigned)p.nsplit, reinterpret_cast<int*>(smem)))
            return;
        splitk_reduce<NC, CF::NT, I8>(slabs, p.nsplit, split, tid, v);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const AccT4 w = bitcast<AccT4>(v[((b * FN + i) * FM + j) * 4 + q]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[b][i][j][4 * q + e] = w[e];
                    }
    }

    // ---- epilogue: lane row m, runs of 4 columns ----
    // Everything the epilogue reads (row / column scales, C for beta) is
    // loaded before the first store, from clamped addresses: a load issued
    // after a store to memory the compiler cannot tell apart waits for it, one
    // round trip per run of 4 columns.
    unsigned char* Cb = static_cast<unsigned char*>(p.C) + batch * p.sC * (OUT == kI8Acc32 ? 4 : 2);
    float sav[FM];
    float sbv[FN][4][4];
    u32x2 oldc[FM][FN][4];
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int mc = min(m0 + wm * 32 * FM + 32 * j + l32, M - 1);
        sav[j] = 1.0f;
        if constexpr (OUT == kI8RowCol) sav[j] = h2f(p.sa[mc]);
        if constexpr (OUT == kF16AlphaBeta) {
            if (p.beta != 0.0f) {
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (CF::KW > 1 && q / NQ != kw) continue;
                        const int nc = min(n0 + wn * 32 * FN + 32 * i + 8 * q + 4 * kh, N - 4);
                        oldc[j][i][q] =
                            *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(Cb) + (int64_t)mc * N + nc);
                    }
            }
        }
    }
    if constexpr (OUT == kI8RowCol) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int nc = min(n0 + wn * 32 * FN + 32 * i + 8 * q + 4 * kh, N - 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) sbv[i][q][e] = h2f(p.sb[nc + e]);
            }
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * 32 * FM + 32 * j + l32;
        if (m >= M) continue;
        const float sa = sav[j];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (CF::KW > 1 && q / NQ != kw) continue;
                const int n = n0 + wn * 32 * FN + 32 * i + 8 * q + 4 * kh;
                if (n >= N) continue;  // N % 8 == 0: the run is whole
                if constexpr (OUT == kI8Acc32) {
                    int* dst = reinterpret_cast<int*>(Cb) + (int64_t)m * N + n;
                    *reinterpret_cast<i32x4*>(dst) =
                        i32x4{acc[0][i][j][4 * q], acc[0][i][j][4 * q + 1], acc[0][i][j][4 * q + 2], acc[0][i][j][4 * q + 3]};
                } else {
                    uint16_t* dst = reinterpret_cast<uint16_t*>(Cb) + (int64_t)m * N + n;
                    float r[4];
                    if constexpr (OUT == kF16AlphaBeta) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = p.alpha * acc[0][i][j][4 * q + e];
                        if (p.beta != 0.0f) {
                            const u32x2 c = oldc[j][i][q];
                            r[0] = fmaf(p.beta, h2f(c.x & 0xffffu), r[0]);
                            r[1] = fmaf(p.beta, h2f(c.x >> 16), r[1]);
                            r[2] = fmaf(p.beta, h2f(c.y & 0xffffu), r[2]);
                            r[3] = fmaf(p.beta, h2f(c.y >> 16), r[3]);
                        }
                    } else if constexpr (OUT == kF16SwiGLU) {
                        // gate and up rounded to fp16 as two GEMM outputs would be
                        const uint16_t o0 = swiglu_h(f2h(acc[0][i][j][4 * q]), f2h(acc[NB - 1][i][j][4 * q]));
                        const uint16_t o1 = swiglu_h(f2h(acc[0][i][j][4 * q + 1]), f2h(acc[NB - 1][i][j][4 * q + 1]));
                        const uint16_t o2 = swiglu_h(f2h(acc[0][i][j][4 * q + 2]), f2h(acc[NB - 1][i][j][4 * q + 2]));
                        const uint16_t o3 = swiglu_h(f2h(acc[0][i][j][4 * q + 3]), f2h(acc[NB - 1][i][j][4 * q + 3]));
                        *reinterpret_cast<u32x2*>(dst) = u32x2{(unsigned)o0 | ((unsigned)o1 << 16),
                                                               (unsigned)o2 | ((unsigned)o3 << 16)};
                        continue;
                    } else if constexpr (OUT == kI8Tensor) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = static_cast<float>(acc[0][i][j][4 * q + e]) * p.scale;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = static_cast<float>(acc[0][i][j][4 * q + e]) * (sa * sbv[i][q][e]);
                    }
                    *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(r[0], r[1]), pack2h(r[2], r[3])};
                }
            }
    }
}

}  // namespace sk
}  // namespace clove
