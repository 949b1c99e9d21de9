// INT8 GEMM for large shapes on gfx950: the FP16 256x256 kernel
// (f16_dma_gemm.hpp) on int8 operands.
//
//   acc[m, n] = sum_k A[m, k] * B[k, n]        int8 x int8 -> int32 (exact)
//   C = fp16(acc * scale) | fp16(acc * (sa[m] * sb[n])) | acc (int32)
//
// Requirements (checked by the host): zero points 0, K % 128 == 0, N % 16 == 0,
// A / B / C 16-byte aligned, operands < 2^31 bytes.  Ragged M and N as in the
// FP16 kernel: rows past the end read as zero through the buffer range check,
// columns past N only reach outputs that are never stored.
//
// A K tile is 128 bytes of k, the same bytes per stage as the FP16 kernel's
// 64 fp16 k, so the stage sizes, the DMA plan and the MFMA / fragment-read slot
// plan (kPlan) are the FP16 kernel's, with two k-steps of 64 k per tile on
// v_mfma_i32_16x16x64_i8:
//   A  256 rows x 128 B, chunk c of row r at slot c ^ (r % 8) ^ ((r / 8) % 2);
//      lane (q, h) of fragment x, k-step s reads row 16 x + q, chunk 4 s + h:
//      k = 64 s + 16 h .. + 15
//   B  128 k-rows x 256 B (N-contiguous), chunk c of row r at slot c ^ (r % 8).
//      ds_read_b64_tr_b8: within a 16-lane group, result lane j byte r = source
//      lane 2 r + j / 8 byte j % 8; with source lane q pointing at 8 bytes of
//      k-row kb + q / 2, columns 16 i + 8 (q % 2), result lane j receives
//      k = kb .. kb + 7 of column 16 i + j.  Two reads (kb = 64 s + 16 h + 8 e,
//      e = 0, 1) give the same 16 k as the A lane of group h.
// The eight rows of one read group land in eight different slots, so every
// fragment read is bank-conflict free.
#pragma once

#include "common.hpp"
#include "f16_dma_gemm.hpp"

namespace clove {
namespace i8big {

using namespace hw;
using dma::dma16;
using dma::make_rsrc;
using dma::stage_barrier;
using dma::vmcnt_imm;

enum Out { kTensor = 1, kRowCol = 2, kAcc32 = 3 };

struct Args {
    const int8_t* A;
    const int8_t* B;
    void* C;             // fp16 [M, N], or int32 for kAcc32
    const uint16_t* sa;  // [M] fp16 (kRowCol)
    const uint16_t* sb;  // [N] fp16 (kRowCol)
    float scale;         // kTensor
    int M, N, K;
    int tiles_m, tiles_n;
};

struct Cfg {
    static constexpr int BM = 256, BN = 256, BKB = 128, NW = 4, NT = 256;  // BKB: k (bytes) per tile
    static constexpr int WTM = 128, WTN = 128, FM = 8, FN = 8;
    static constexpr int A_BYTES = BM * BKB, B_BYTES = BKB * BN;
    static constexpr int A_STAGES = 3, B_STAGES = 2;
    static constexpr int LDS_BYTES = A_STAGES * A_BYTES + B_STAGES * B_BYTES;
    static constexpr int DMA_A = A_BYTES / 1024 / NW, DMA_B = B_BYTES / 1024 / NW;
    static_assert(LDS_BYTES <= 163840, "LDS");
    static_assert(NW * WTM * (WTN * 2 + 16) <= LDS_BYTES, "epilogue staging");
    static_assert(DMA_A == dma::Big::DMA_A && DMA_B == dma::Big::DMA_B, "the FP16 kernel's DMA plan");
};

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef int i32x2v __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) i32x2v lds_i32x2v;

// the accumulators' wait states around the inline-asm MFMAs (see the FP16 kernel)
template <int NOPS>
__device__ __forceinline__ void acc_fence(i32x4 (&acc)[64]) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        i32x4* a = acc + 8 * g;
        if (g == 0 && NOPS > 0)
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
        else
            asm volatile("s_nop 1"
                         : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
    }
}

template <int OUT>
__global__ void __launch_bounds__(Cfg::NT) gemm_i8_big(Args p) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BKB = Cfg::BKB, NW = Cfg::NW;
    constexpr int WTM = Cfg::WTM, WTN = Cfg::WTN, FM = Cfg::FM, FN = Cfg::FN;
    constexpr int A_BYTES = Cfg::A_BYTES, B_BYTES = Cfg::B_BYTES;
    using dma::kBar;
    using dma::kPlan;
    using dma::kWaitBar;
    using dma::plan_dma_a;
    using dma::plan_dma_b;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[Cfg::LDS_BYTES / 2];

    int tm, tn;
    {
        // workgroups are dealt to the 8 XCDs round-robin: each XCD gets a
        // contiguous range of tiles, walked 8 tile-rows at a time
        int bid = blockIdx.x;
        const int nblk = gridDim.x;
        if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
        constexpr int GM = 8;
        const int group = bid / (GM * p.tiles_n);
        const int first_m = group * GM;
        const int gm = min(p.tiles_m - first_m, GM);
        const int in_group = bid - group * GM * p.tiles_n;
        tm = first_m + in_group % gm;
        tn = in_group / gm;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;
    const int KT = K / BKB;

    const u32x4 ra = make_rsrc(p.A, (unsigned)M * K);
    const u32x4 rb = make_rsrc(p.B, (unsigned)K * N);
    const unsigned lds_base = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) uint16_t*)smem));
    const unsigned lds_a = lds_base, lds_b = lds_base + Cfg::A_STAGES * A_BYTES;

    // ---- A DMA: instruction i of wave w fills rows 32 i + 8 w + lane / 8,
    // slot lane % 8, which holds global chunk slot ^ swz(row) ----
    const int offA = (m0 + 8 * wave + (lane >> 3)) * K + 16 * ((lane & 7) ^ (lane >> 3) ^ (wave & 1));
    auto dma_a = [&](int kt, int ast, int i) {
        dma16(ra, lds_a + ast * A_BYTES + (i * NW + wave) * 1024, offA, kt * BKB + i * 32 * K);
    };
    // ---- B DMA: instruction i of wave w fills k-rows 16 i + 4 w + lane / 16,
    // slot lane % 16 (256-byte rows), which holds global chunk slot ^ (row % 8) ----
    const int rB = 4 * wave + (lane >> 4);
    const int offB = rB * N + n0 + 16 * ((lane & 15) ^ (rB & 7));
    auto dma_b = [&](int kt, int bst, int i) {
        dma16(rb, lds_b + bst * B_BYTES + (16 * i + 4 * wave) * 256, offB, (kt * BKB + 16 * i) * N);
    };

    // ---- A fragment x of k-step s ----
    const int q = lane & 15, h = lane >> 4;
    unsigned fo[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) fo[s] = wm * WTM * BKB + q * BKB + 16 * ((4 * s + h) ^ (q & 7) ^ (q >> 3));
    auto rd_a = [&](int ast, int s, int x) -> u32x4 {
        return *reinterpret_cast<const lds_u32x4*>((size_t)(lds_a + ast * A_BYTES + fo[s] + x * 16 * BKB));
    };
    // ---- B fragment i (columns wn 128 + 16 i ..), k-step s, read e: source
    // lane q of group h points at k-row 64 s + 16 h + 8 e + q / 2, bytes
    // 16 i + 8 (q % 2) of the wave's columns, at slot (wn 8 + i) ^ (q / 2) ----
    unsigned tb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) tb[i] = (16 * h + (q >> 1)) * 256 + 128 * wn + 16 * (i ^ (q >> 1)) + 8 * (q & 1);
    auto rd_b = [&](unsigned base, int s, int i, int e) -> u32x2 {
        const unsigned a = base + tb[i] + (64 * s + 8 * e) * 256;
        const i32x2v v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_i32x2v*>((size_t)a));
        return u32x2{(unsigned)v[0], (unsigned)v[1]};
    };

    i32x4 acc[FN * FM];  // tile (i, j) at 8 i + j
#pragma unroll
    for (int n = 0; n < FN * FM; ++n) acc[n] = i32x4{0, 0, 0, 0};
    u32x4 fa[2][FM];
    u32x2 fb[FN][2];

    // ---- prologue: A(0), B(0), A(1), B(1) in flight in that order, the first
    // two landed, k-step 0 fragments of tile 0 ----
#pragma unroll
    for (int i = 0; i < Cfg::DMA_A; ++i) dma_a(0, 0, i);
#pragma unroll
    for (int i = 0; i < Cfg::DMA_B; ++i) dma_b(0, 0, i);
    const int k1 = min(1, KT - 1);
#pragma unroll
    for (int i = 0; i < Cfg::DMA_A; ++i) dma_a(k1, 1, i);
#pragma unroll
    for (int i = 0; i < Cfg::DMA_B; ++i) dma_b(k1, 1, i);
    stage_barrier<vmcnt_imm(Cfg::DMA_A + Cfg::DMA_B)>();
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        fa[0][x] = rd_a(0, 0, x);
        fb[x][0] = rd_b(lds_b, 0, x, 0);
        fb[x][1] = rd_b(lds_b, 0, x, 1);
    }
    acc_fence<0>(acc);

    int ast = 0;
    auto tile = [&](int kt, auto PC) {
        constexpr int P = decltype(PC)::value;
        const int ast1 = ast == 2 ? 0 : ast + 1;
        const int ast2 = ast1 == 2 ? 0 : ast1 + 1;
        const int k2 = min(kt + 2, KT - 1);
        unsigned bcur = lds_b + P * B_BYTES, bnext = lds_b + (P ^ 1) * B_BYTES;
        asm volatile("" : "+v"(bcur), "+v"(bnext));
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int n = 0; n < 64; ++n) {
                const int g = 64 * s + n;
                if (g == kBar) stage_barrier<vmcnt_imm(kWaitBar)>();
                {
                    const int i = n >> 3, j = n & 7;
                    const u32x4 bf = {fb[i][0].x, fb[i][0].y, fb[i][1].x, fb[i][1].y};
                    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0"
                                 : "+a"(acc[n])
                                 : "v"(bf), "v"(fa[s][j]));
                }
                const int op = kPlan.op[g];
                if (op >= 0) {
                    const int kind = op >> 5, x = (op >> 1) & 15, e = op & 1;
                    if (kind == dma::kA1) fa[1][x] = rd_a(ast, 1, x);
                    else if (kind == dma::kB1) fb[x][e] = rd_b(bcur, 1, x, e);
                    else if (kind == dma::kB0) fb[x][e] = rd_b(bcur, 0, x, e);
                    else if (kind == dma::kA0n) fa[0][x] = rd_a(ast1, 0, x);
                    else fb[x][e] = rd_b(bnext, 0, x, e);
                }
                if (plan_dma_a(g) >= 0) dma_a(k2, ast2, plan_dma_a(g));
                if (plan_dma_b(g) >= 0) dma_b(k2, P, plan_dma_b(g));
                __builtin_amdgcn_sched_barrier(0);
            }
        ast = ast1;
    };
    int kt = 0;
#pragma unroll 1
    for (; kt + 1 < KT; kt += 2) {
        tile(kt, dma::IntC<0>{});
        tile(kt + 1, dma::IntC<1>{});
    }
    if (kt < KT) tile(kt, dma::IntC<0>{});
    stage_barrier<vmcnt_imm(0)>();
    acc_fence<1>(acc);

    // lane holds m = 16 j + q, n = 16 i + 4 h + 0..3 of tile (i, j)
    const int wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;
    if constexpr (OUT == kAcc32) {
        int* C = static_cast<int*>(p.C);
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int gm = wrow0 + 16 * j + q;
            if (gm >= M) continue;
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int gn = wcol0 + 16 * i + 4 * h;
                if (gn < N) *reinterpret_cast<i32x4*>(C + (int64_t)gm * N + gn) = acc[8 * i + j];
            }
        }
        return;
    }
    // fp16 outputs: every scale loaded first (clamped addresses), the tile
    // converted into LDS, then whole 16-byte row segments stored
    float sa[FM], sb[FN][4];
#pragma unroll
    for (int j = 0; j < FM; ++j) sa[j] = OUT == kRowCol ? h2f(p.sa[min(wrow0 + 16 * j + q, M - 1)]) : p.scale;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) sb[i][e] = OUT == kRowCol ? h2f(p.sb[min(wcol0 + 16 * i + 4 * h + e, N - 1)]) : 1.0f;
    constexpr int PITCH = WTN * 2 + 16;
    const unsigned wbase = lds_base + wave * WTM * PITCH;
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const i32x4 v = acc[8 * i + j];
            float r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                r[e] = OUT == kRowCol ? static_cast<float>(v[e]) * (sa[j] * sb[i][e]) : static_cast<float>(v[e]) * sa[j];
            const u32x2 w = {pack2h(r[0], r[1]), pack2h(r[2], r[3])};
            *reinterpret_cast<lds_u32x2*>((size_t)(wbase + (16 * j + q) * PITCH + (16 * i + 4 * h) * 2)) = w;
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes are visible to its reads
    uint16_t* C = static_cast<uint16_t*>(p.C);
    constexpr int CPRW = WTN / 8, RPI = 64 / CPRW;
#pragma unroll
    for (int it = 0; it < WTM / RPI; ++it) {
        const int m = it * RPI + lane / CPRW, c = lane % CPRW;
        const u32x4 v = *reinterpret_cast<const lds_u32x4*>((size_t)(wbase + m * PITCH + c * 16));
        const int gm = wrow0 + m, gn = wcol0 + 8 * c;
        // nontemporal, as in the FP16 kernel: no dirty C in L2 at the kernel's end
        if (gm < M && gn < N) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + (int64_t)gm * N + gn));
    }
}

}  // namespace i8big
}  // namespace clove
