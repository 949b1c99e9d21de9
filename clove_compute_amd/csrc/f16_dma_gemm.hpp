// FP16 GEMM for large, aligned shapes on gfx950.
//
//   C[M,N] = alpha * A[M,K] @ B[K,N] + beta * C      fp32 accumulation
//
// Requirements (checked by the host): K % 64 == 0, N % 8 == 0, M >= 1, N >= 8,
// A/B/C 16-byte aligned, each operand < 2^31 bytes.  Ragged M and N are
// handled by the buffer range check (rows past the end of A and B read as
// zero) and by masking the stores; columns past N inside B's last tile read
// neighbouring data that only reaches outputs that are never stored.
//
// Tiling.  A 256x256 output tile per workgroup, 4 waves of 128x128, K in tiles
// of 64.  Each wave's 128x128 is an 8x8 grid of v_mfma_f32_16x16x32_f16: at
// equal flops this shape reads and writes a quarter of the accumulator bytes
// of the 32x32x16 form per instruction, and on this part the clock, not the
// instruction count, bounds a 4096^3 GEMM (the same loop runs ~15 % faster in
// wall time with it, at the same cycles per flop).
//
// Data movement.  Both operands go HBM -> LDS by LDS DMA (buffer_load_dwordx4
// ... lds): no VGPR staging, no register transpose and no ds_write in the main
// loop.  A is stored K-contiguous ([m][64 k], 128-byte rows) and its MFMA
// fragments are ds_read_b128; B stays N-contiguous ([k][256 n], 512-byte rows)
// and its fragments come from the transposing read ds_read_b64_tr_b16: within
// a 16-lane group, result lane j element r = source lane 4r + j/4 element
// j%4, so with source lane s pointing at 8 bytes of k-row kb + s/4, columns
// 4(s%4)..+3, every lane receives 4 consecutive k of one column; two such
// reads make the 8-k operand.  Both layouts XOR-swizzle their 16-byte chunks
// so that every fragment read is bank-conflict free:
//   A row r: chunk c at slot c ^ (r % 8) ^ ((r / 8) % 2)
//   B row r: chunk c at slot c ^ 2 (r % 4)
//
// Pipeline.  LDS holds three A stages and two B stages (160 KB).  Tile kt's A
// arrives during tile kt-2, its B during tile kt-1 right after that tile's
// barrier (which frees the B stage of tile kt-1); one workgroup barrier per K
// tile, three quarters of the way through it.  MFMAs, fragment reads and DMAs
// follow a fixed slot plan (kPlan below): one LDS read every 2-3 MFMAs, so the
// LDS pipe, shared by the four waves, runs at an even ~75 % instead of in
// bursts.  DMA completion is tracked with explicit vmcnt waits (the DMAs are
// inline asm, so the compiler neither waits for them before every LDS read nor
// counts them).
//
// Accumulators.  The MFMAs are inline asm with the accumulator tied in place
// ("+a"): the compiler's own MFMA selection copied accumulator tuples between
// registers around the unrolled loop (hundreds of v_accvgpr moves per tile).
// Since the compiler does not see these as MFMAs, the kernel inserts the
// wait states its hazard recognizer would: before the first MFMA reads the
// zeroed accumulators and after the last MFMA, before they are read.
//
// Epilogue (beta == 0): each wave's fp16 tile goes through LDS so that every
// global store is a full 16-byte lane of a contiguous row segment.
#pragma once

#include "common.hpp"

namespace clove {
namespace dma {

using namespace hw;

struct Args {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    int M, N, K;
    float alpha, beta;
    int64_t sA, sB, sC;  // batch strides (elements)
    int tiles_m, tiles_n;
    // the K split (gemm_f16_big_split, one batch): workgroup r takes K tiles
    // [s ktps, (s + 1) ktps) of tile r / nsplit, s = r % nsplit, publishes its
    // fp32 partial tile to `part` (slab r) and counts in `counters` (one per
    // tile); the last to arrive sums the partials in split order and stores
    // the tile
    int nsplit, ktps;
    float* part;
    unsigned* counters;
};

// s_waitcnt with only the vector-memory counter constrained
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14);
}

// One 16-byte-per-lane LDS DMA: buffer_load_dwordx4 ... lds writes lane l's
// 16 bytes at LDS byte address m0 + 16 l.  Issued as inline asm so that the
// compiler does not treat it as a possible writer of the stage being read
// (it would otherwise wait for every DMA in flight before each LDS read);
// completion is tracked explicitly with vmcnt + a workgroup barrier.
// The compiler does not see an LDS DMA inside the asm, so the asm carries the
// wait state an LDS DMA needs after the SALU write of M0 that the "{m0}"
// operand places right in front of it (the build's hazard scan checks it).
__device__ __forceinline__ void dma16(const u32x4& rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
                 : "memory");
}

// raw buffer resource over [base, base + bytes): stride 0, dword3 as for gfx9
// global memory (32-bit data format, no swizzle)
__device__ __forceinline__ u32x4 make_rsrc(const void* base, unsigned bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    u32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((unsigned)a);
    r.y = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32) & 0xffffu);
    r.z = bytes;
    r.w = 0x00020000u;
    return r;
}

// all waves: own DMAs up to the last `n` issued have landed, LDS reads
// returned, then the workgroup barrier; the empty asm statements keep the
// compiler from moving LDS accesses across it
template <int IMM>
__device__ __forceinline__ void stage_barrier() {
    __builtin_amdgcn_s_waitcnt(IMM);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int V>
struct IntC {
    static constexpr int value = V;
};

// ---------------------------------------------------------------------------
// Tile configuration and slot plan
// ---------------------------------------------------------------------------
struct Big {
    static constexpr int BM = 256, BN = 256, BK = 64, NW = 4, NT = 256;
    static constexpr int WTM = 128, WTN = 128, FM = 8, FN = 8;  // 16x16 fragments per wave
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
    static constexpr int A_STAGES = 3, B_STAGES = 2;
    static constexpr int LDS_BYTES = A_STAGES * A_BYTES + B_STAGES * B_BYTES;
    static constexpr int DMA_A = A_BYTES / 1024 / NW, DMA_B = B_BYTES / 1024 / NW;  // per wave per tile
    static_assert(LDS_BYTES <= 163840, "LDS");
    static_assert(NW * WTM * (WTN * 2 + 16) <= LDS_BYTES, "epilogue staging");
    static_assert(DMA_A == 8 && DMA_B == 8, "slot plan");
};

// A K tile is 128 MFMA slots: k-step 0 (32 k) in slots 0..63, k-step 1 in
// 64..127; MFMA n of a k-step is tile (i = n / 8, j = n % 8), B fragment i x
// A fragment j.  Registers: fa[s][8] (A, one set per k-step) and fb[8] (B,
// two halves each) refilled as slots free them: fb[i] is last used at slot
// 8i + 7 of each k-step.  The barrier sits before slot kBar.
enum ReadKind : int {
    kA1 = 1,   // fa[1][i]: A, k-step 1 of this tile
    kB1 = 2,   // fb[i] half e: B, k-step 1 of this tile
    kB0 = 3,   // fb[i] half e: B, k-step 0 of this tile (still in use at the previous barrier)
    kA0n = 4,  // fa[0][i]: A, k-step 0 of the next tile (after the barrier)
    kB0n = 5,  // fb[i] half e: B, k-step 0 of the next tile (after the barrier)
};
struct ReadSlot {
    int slot, kind, i, e;
};
constexpr int kBar = 96;
// 48 LDS reads per wave per tile, evenly spaced (one per 2-3 MFMAs), each no
// earlier than its register frees and at least 8 slots before its first use
constexpr ReadSlot kReads[48] = {
    {0, kB0, 2, 0}, {2, kB0, 2, 1}, {5, kB0, 3, 0}, {8, kB0, 3, 1}, {10, kB0, 4, 0},
    {13, kB0, 4, 1}, {16, kB0, 5, 0}, {18, kB0, 5, 1}, {21, kB0, 6, 0}, {24, kB0, 6, 1},
    {26, kB0, 7, 0}, {29, kB0, 7, 1}, {32, kA1, 0, 0}, {34, kB1, 0, 0}, {37, kB1, 0, 1},
    {40, kA1, 1, 0}, {42, kA1, 2, 0}, {45, kA1, 3, 0}, {48, kA1, 4, 0}, {50, kA1, 5, 0},
    {53, kA1, 6, 0}, {56, kA1, 7, 0}, {58, kB1, 1, 0}, {61, kB1, 1, 1}, {64, kB1, 2, 0},
    {66, kB1, 2, 1}, {69, kB1, 3, 0}, {72, kB1, 3, 1}, {74, kB1, 4, 0}, {77, kB1, 4, 1},
    {80, kB1, 5, 0}, {82, kB1, 5, 1}, {85, kB1, 6, 0}, {88, kB1, 6, 1}, {90, kB1, 7, 0},
    {93, kB1, 7, 1}, {96, kA0n, 0, 0}, {98, kB0n, 0, 0}, {101, kB0n, 0, 1},
    {104, kA0n, 1, 0}, {106, kA0n, 2, 0}, {109, kA0n, 3, 0}, {112, kA0n, 4, 0},
    {114, kA0n, 5, 0}, {117, kA0n, 6, 0}, {120, kA0n, 7, 0}, {122, kB0n, 1, 0},
    {125, kB0n, 1, 1}};

// DMAs per tile: A of tile kt+2 before the barrier, B of tile kt+2 after it
// (into the B stage the barrier just freed)
__host__ __device__ constexpr int plan_dma_a(int g) { return (g >= 4 && g < kBar && (g - 4) % 12 == 0) ? (g - 4) / 12 : -1; }
__host__ __device__ constexpr int plan_dma_b(int g) { return (g >= 98 && (g - 98) % 4 == 0) ? (g - 98) / 4 : -1; }
// At the barrier of tile kt, A(kt+1) and B(kt+1) (issued during tile kt-1,
// B last) must have landed: only this tile's A DMAs may still be in flight.
constexpr int kWaitBar = 8;

struct PlanTable {
    short op[128];  // kind * 32 + i * 2 + e, or -1
};
constexpr PlanTable make_plan_table() {
    PlanTable t{};
    for (int g = 0; g < 128; ++g) t.op[g] = -1;
    for (const ReadSlot& r : kReads) t.op[r.slot] = (short)(r.kind * 32 + r.i * 2 + r.e);
    return t;
}
constexpr PlanTable kPlan = make_plan_table();

// Every fragment read exactly once per tile, each inside its window; the DMA
// plan issues 8 + 8 per tile with the A DMAs before the barrier and the B
// DMAs after it.
constexpr bool plan_valid() {
    int seen[6][8][2] = {};
    int slots[128] = {};
    for (const ReadSlot& r : kReads) {
        if (r.slot < 0 || r.slot >= 128 || slots[r.slot]++) return false;
        if (r.i < 0 || r.i >= 8 || r.e < 0 || r.e > 1) return false;
        seen[r.kind][r.i][r.e]++;
        const int s = r.slot, i = r.i;
        switch (r.kind) {
            case kA1: if (r.e != 0 || s > 64 + i - 8) return false; break;
            case kB1: if (s < 8 * i + 8 || s > 64 + 8 * i - 8) return false; break;
            case kB0: if (i < 2 || s > 8 * i - 8) return false; break;
            case kA0n: if (r.e != 0 || s < kBar || s > 128 + i - 6) return false; break;
            case kB0n: if (i >= 2 || s < kBar || s < 64 + 8 * i + 8 || s > 128 + 8 * i - 6) return false; break;
            default: return false;
        }
    }
    for (int i = 0; i < 8; ++i) {
        if (seen[kA1][i][0] != 1 || seen[kA0n][i][0] != 1) return false;
        for (int e = 0; e < 2; ++e)
            if (seen[kB1][i][e] != 1 || seen[i < 2 ? kB0n : kB0][i][e] != 1) return false;
    }
    int na = 0, nb = 0;
    for (int g = 0; g < 128; ++g) {
        if (plan_dma_a(g) >= 0) { if (g >= kBar || plan_dma_a(g) != na) return false; ++na; }
        if (plan_dma_b(g) >= 0) { if (g <= kBar || plan_dma_b(g) != nb) return false; ++nb; }
    }
    return na == Big::DMA_A && nb == Big::DMA_B && na == kWaitBar;
}
static_assert(plan_valid(), "slot plan");

// tile `tile` of one batch: the tiles are walked 8 tile-rows at a time
__device__ __forceinline__ void tile_rc(const Args& p, int tile, int& tm, int& tn) {
    constexpr int GM = 8;
    const int group = tile / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gm = min(p.tiles_m - first_m, GM);
    const int in_group = tile - group * GM * p.tiles_n;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

__device__ __forceinline__ void tile_coords(const Args& p, int& batch, int& tm, int& tn) {
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    // workgroups are dealt to the 8 XCDs round-robin: give each XCD a
    // contiguous range of tiles so its L2 sees shared A and B panels
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int per_batch = p.tiles_m * p.tiles_n;
    batch = bid / per_batch;
    tile_rc(p, bid - batch * per_batch, tm, tn);
}

typedef short i16x4v __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) i16x4v lds_i16x4v;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

// The accumulators as inline-asm operands, 8 tiles at a time: the wait states
// (s_nop) a VALU write / MFMA result needs before the next reader, placed
// where the compiler cannot move the readers or writers across them.
template <int NOPS>
__device__ __forceinline__ void acc_fence(f32x4 (&acc)[64]) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        f32x4* a = acc + 8 * g;
        if (g == 0 && NOPS > 0)
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
        else
            asm volatile("s_nop 1"
                         : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
    }
}

// Per-workgroup phase timestamps of the TS instantiation (one record of
// kTsWords 64-bit words per workgroup, written by wave 0 at the end): shader
// cycles (s_memtime) and the constant 100 MHz clock (s_memrealtime) at
// entry, once the first K tile has landed, after the first two K tiles, after
// the last K tile and once the output stores have completed; then the
// workgroup's tile count, HW_ID and XCC_ID.
constexpr int kTsWords = 16;
enum TsSlot : int { kTsEntry = 0, kTsFirst = 2, kTsTwo = 4, kTsLoop = 6, kTsEnd = 8, kTsKT = 10, kTsHw = 11 };

// The kernel body.  TS = false is the product kernel; TS = true (bench.py's
// phase breakdown) adds the timestamps above and nothing else: the
// s_memtime / s_memrealtime reads at the phase boundaries (whose results the
// compiler waits for with the LDS reads in flight at that point) and one
// store per workgroup after the output stores.
template <class CF, bool TS, bool SPLIT = false>
__device__ __forceinline__ void big_body(const Args& p, unsigned long long* ts) {
    using Big = CF;
    unsigned long long tsv[10] = {};
    if constexpr (TS) {
        tsv[kTsEntry] = __builtin_amdgcn_s_memtime();
        tsv[kTsEntry + 1] = __builtin_amdgcn_s_memrealtime();
    }
    constexpr int BM = Big::BM, BN = Big::BN, BK = Big::BK, NW = Big::NW;
    constexpr int WTM = Big::WTM, WTN = Big::WTN, FM = Big::FM, FN = Big::FN;
    constexpr int A_BYTES = Big::A_BYTES, B_BYTES = Big::B_BYTES;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[Big::LDS_BYTES / 2];

    const int M = p.M, N = p.N, K = p.K;
    const int KT = K / BK;
    int batch, tm, tn;
    // this workgroup's K tiles [kbeg, kend); SPLIT: part `split` of tile rtile
    int kbeg = 0, kend = KT, rtile = -1, split = 0;
    if constexpr (SPLIT) {
        const int r = blockIdx.x;
        batch = 0;
        rtile = r / p.nsplit;
        split = r - rtile * p.nsplit;
        tile_rc(p, rtile, tm, tn);
        kbeg = split * p.ktps;
        kend = min(KT, kbeg + p.ktps);
    } else {
        tile_coords(p, batch, tm, tn);
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = tm * BM, n0 = tn * BN;

    const u32x4 ra = make_rsrc(p.A + batch * p.sA, (unsigned)M * K * 2);
    const u32x4 rb = make_rsrc(p.B + batch * p.sB, (unsigned)K * N * 2);
    const unsigned lds_base = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) uint16_t*)smem));
    const unsigned lds_a = lds_base, lds_b = lds_base + Big::A_STAGES * A_BYTES;

    // ---- A DMA: instruction i of wave w fills rows 32 i + 8 w + lane / 8,
    // slot lane % 8, which holds global chunk slot ^ swz(row) ----
    const int offA = 2 * ((m0 + 8 * wave + (lane >> 3)) * K + 8 * ((lane & 7) ^ (lane >> 3) ^ (wave & 1)));
    auto dma_a = [&](int kt, int ast, int i) {
        dma16(ra, lds_a + ast * A_BYTES + (i * NW + wave) * 1024, offA, kt * BK * 2 + i * 32 * K * 2);
    };
    // ---- B DMA: instruction i of wave w fills k-rows 8 i + 2 w + lane / 32,
    // slot lane % 32 (512-byte rows) ----
    const int rB = 2 * wave + (lane >> 5);
    const int offB = 2 * (rB * N + n0) + 16 * ((lane & 31) ^ (2 * (rB & 3)));
    auto dma_b = [&](int kt, int bst, int i) {
        dma16(rb, lds_b + bst * B_BYTES + (8 * i + 2 * wave) * 512, offB, (kt * BK + 8 * i) * N * 2);
    };

    // ---- A fragment x of k-step s: row 16 x + q, chunk 4 s + h, at slot
    // (4 s + h) ^ (q % 8) ^ (q / 8) (q = lane % 16, h = lane / 16) ----
    const int q = lane & 15, h = lane >> 4;
    unsigned fo[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) fo[s] = wm * WTM * BK * 2 + q * BK * 2 + 16 * ((4 * s + h) ^ (q & 7) ^ (q >> 3));
    auto rd_a = [&](int ast, int s, int x) -> f16x8 {
        return bitcast<f16x8>(
            *reinterpret_cast<const lds_u32x4*>((size_t)(lds_a + ast * A_BYTES + fo[s] + x * 16 * BK * 2)));
    };
    // ---- B fragment i (columns wn 128 + 16 i ..), k-step s, half e: source lane
    // q of group h points at k-row 32 s + 8 h + 4 e + q / 4, columns + 4 (q % 4);
    // its slot (chunk ^ 2 (q / 4)) depends on i % 4 only, i / 4 adds 128 bytes ----
    const int t4 = q >> 2;
    unsigned tb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        tb[u] = (8 * h + t4) * 512 + 16 * (wn * 16 + ((2 * u + ((q & 3) >> 1)) ^ (2 * t4))) + 8 * (q & 1);
    auto rd_b = [&](unsigned base, int s, int i, int e) -> u32x2 {
        const unsigned a = base + tb[i & 3] + (32 * s + 4 * e) * 512 + 128 * (i >> 2);
        return bitcast<u32x2>(__builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4v*>((size_t)a)));
    };

    f32x4 acc[FN * FM];  // tile (i, j) at 8 i + j
#pragma unroll
    for (int n = 0; n < FN * FM; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    f16x8 fa[2][FM];
    u32x2 fb[FN][2];

    // ---- prologue: A(kbeg), B(kbeg), A(kbeg + 1), B(kbeg + 1) in flight in that
    // order (the waits below count on it), the first two landed, k-step 0
    // fragments of tile kbeg ----
#pragma unroll
    for (int i = 0; i < Big::DMA_A; ++i) dma_a(kbeg, 0, i);
#pragma unroll
    for (int i = 0; i < Big::DMA_B; ++i) dma_b(kbeg, 0, i);
    const int k1 = min(kbeg + 1, kend - 1);
#pragma unroll
    for (int i = 0; i < Big::DMA_A; ++i) dma_a(k1, 1, i);
#pragma unroll
    for (int i = 0; i < Big::DMA_B; ++i) dma_b(k1, 1, i);
    stage_barrier<vmcnt_imm(Big::DMA_A + Big::DMA_B)>();
    if constexpr (TS) {
        tsv[kTsFirst] = __builtin_amdgcn_s_memtime();
        tsv[kTsFirst + 1] = __builtin_amdgcn_s_memrealtime();
    }
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        fa[0][x] = rd_a(0, 0, x);
        fb[x][0] = rd_b(lds_b, 0, x, 0);
        fb[x][1] = rd_b(lds_b, 0, x, 1);
    }
    acc_fence<0>(acc);  // the zeroed accumulators are written before the first MFMA reads them

    int ast = 0;  // A stage of the current tile (tiles rotate through 3)
    // tile kt with parity P: B stage P holds it, B stage P ^ 1 the next tile
    auto tile = [&](int kt, auto PC) {
        constexpr int P = decltype(PC)::value;
        const int ast1 = ast == 2 ? 0 : ast + 1;
        const int ast2 = ast1 == 2 ? 0 : ast1 + 1;
        const int k2 = min(kt + 2, kend - 1);
        // opaque per tile, so the B read addresses fold into instruction offsets
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
                    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                                 : "+a"(acc[n])
                                 : "v"(bitcast<f16x8>(bf)), "v"(fa[s][j]));
                }
                const int op = kPlan.op[g];
                if (op >= 0) {
                    const int kind = op >> 5, x = (op >> 1) & 15, e = op & 1;
                    if (kind == kA1) fa[1][x] = rd_a(ast, 1, x);
                    else if (kind == kB1) fb[x][e] = rd_b(bcur, 1, x, e);
                    else if (kind == kB0) fb[x][e] = rd_b(bcur, 0, x, e);
                    else if (kind == kA0n) fa[0][x] = rd_a(ast1, 0, x);
                    else fb[x][e] = rd_b(bnext, 0, x, e);
                }
                if (plan_dma_a(g) >= 0) dma_a(k2, ast2, plan_dma_a(g));
                if (plan_dma_b(g) >= 0) dma_b(k2, P, plan_dma_b(g));
                __builtin_amdgcn_sched_barrier(0);
            }
        ast = ast1;
    };
    int kt = kbeg;
#pragma unroll 1
    for (; kt + 1 < kend; kt += 2) {
        if constexpr (TS) {
            if (kt == 2) {
                tsv[kTsTwo] = __builtin_amdgcn_s_memtime();
                tsv[kTsTwo + 1] = __builtin_amdgcn_s_memrealtime();
            }
        }
        tile(kt, IntC<0>{});
        tile(kt + 1, IntC<1>{});
    }
    if (kt < kend) tile(kt, IntC<0>{});  // odd number of K tiles
    // every DMA has landed and every wave is done with the stages
    stage_barrier<vmcnt_imm(0)>();
    acc_fence<1>(acc);  // the last MFMA results land before the accumulators are read
    if constexpr (SPLIT) {
        {
            // publish this split's partial tile; the last split to arrive sums
            // them in split order and runs the epilogue
            constexpr int NC = FN * FM;
            float* slabs = p.part + (size_t)rtile * p.nsplit * (NC * Big::NT * 4);
            splitk_publish<NC, Big::NT>(slabs + (size_t)split * (NC * Big::NT * 4), tid, acc);
            // (the stages are dead: every DMA was waited for, every read returned)
            if (!splitk_arrive_is_last(p.counters + rtile, (unsigned)p.nsplit, reinterpret_cast<int*>(smem)))
                return;
            // the sum in split order (((p0 + p1) + p2) + ..., every part read
            // back, this split's own too, so that the accumulators are dead
            // here), then the alpha / beta epilogue straight from the sums:
            // lane holds m = 16 j + q, n = 16 i + 4 h + 0..3 of tile (i, j) =
            // chunk 8 i + j.  Two parts: 16 chunks of both per round trip;
            // more: 8 chunks of one part per round trip.
            constexpr int CG = 16;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                slabs, (short)0, p.nsplit * NC * Big::NT * 16, 0x00020000);
            const int wr0 = m0 + wm * WTM, wc0 = n0 + wn * WTN;
            const int qq = lane & 15, hh = lane >> 4;
            auto ld = [&](int sp, int c) {
                return bitcast<f32x4>(
                    __builtin_amdgcn_raw_buffer_load_b128(rs, ((sp * NC + c) * Big::NT + tid) * 16, 0, kCpolSc1));
            };
#pragma unroll
            for (int c0 = 0; c0 < NC; c0 += CG) {
                f32x4 sum[CG];
                if (p.nsplit == 2) {
                    f32x4 t1[CG];
#pragma unroll
                    for (int c = 0; c < CG; ++c) {
                        sum[c] = ld(0, c0 + c);
                        t1[c] = ld(1, c0 + c);
                    }
#pragma unroll
                    for (int c = 0; c < CG; ++c) sum[c] += t1[c];
                } else {
#pragma unroll
                    for (int h8 = 0; h8 < CG; h8 += 8) {
                        for (int sp = 0; sp < p.nsplit; ++sp) {
                            f32x4 t[8];
#pragma unroll
                            for (int c = 0; c < 8; ++c) t[c] = ld(sp, c0 + h8 + c);
#pragma unroll
                            for (int c = 0; c < 8; ++c) sum[h8 + c] = sp == 0 ? t[c] : sum[h8 + c] + t[c];
                        }
                    }
                }
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    const int i = (c0 + c) >> 3, j = (c0 + c) & 7;
                    const int gm = wr0 + 16 * j + qq, gn = wc0 + 16 * i + 4 * hh;
                    if (gm >= M || gn >= N) continue;
                    uint16_t* dst = p.C + (int64_t)gm * N + gn;
                    const f32x4 v = sum[c];
                    float r[4] = {p.alpha * v[0], p.alpha * v[1], p.alpha * v[2], p.alpha * v[3]};
                    if (p.beta != 0.0f) {
                        const u32x2 old = *reinterpret_cast<const u32x2*>(dst);
                        r[0] = fmaf(p.beta, h2f(old.x & 0xffffu), r[0]);
                        r[1] = fmaf(p.beta, h2f(old.x >> 16), r[1]);
                        r[2] = fmaf(p.beta, h2f(old.y & 0xffffu), r[2]);
                        r[3] = fmaf(p.beta, h2f(old.y >> 16), r[3]);
                    }
                    *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(r[0], r[1]), pack2h(r[2], r[3])};
                }
            }
            return;
        }
    }
    if constexpr (TS) {
        tsv[kTsLoop] = __builtin_amdgcn_s_memtime();
        tsv[kTsLoop + 1] = __builtin_amdgcn_s_memrealtime();
    }
    // TS: the end time once this wave's output stores have completed, and the record
    auto ts_end = [&]() {
        if constexpr (TS) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            tsv[kTsEnd] = __builtin_amdgcn_s_memtime();
            tsv[kTsEnd + 1] = __builtin_amdgcn_s_memrealtime();
            if (wave == 0 && lane == 0) {
                unsigned hw, xcc;
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
                asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
                unsigned long long* r = ts + (size_t)blockIdx.x * kTsWords;
#pragma unroll
                for (int i = 0; i < 10; ++i) r[i] = tsv[i];
                r[kTsKT] = (unsigned long long)KT;
                r[kTsHw] = hw;
                r[kTsHw + 1] = xcc;
            }
        }
    };

    uint16_t* C = p.C + batch * p.sC;
    const int wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;
    // lane holds m = 16 j + q, n = 16 i + 4 h + 0..3 of tile (i, j)
    if (p.beta == 0.0f) {
        constexpr int PITCH = WTN * 2 + 16;  // bytes; the pad spreads rows over the banks
        const unsigned wbase = lds_base + wave * WTM * PITCH;
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const f32x4 v = acc[8 * i + j];
                const u32x2 w = {pack2h(p.alpha * v[0], p.alpha * v[1]), pack2h(p.alpha * v[2], p.alpha * v[3])};
                *reinterpret_cast<lds_u32x2*>((size_t)(wbase + (16 * j + q) * PITCH + (16 * i + 4 * h) * 2)) = w;
            }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes are visible to its reads
        constexpr int CPRW = WTN / 8;          // 16-byte chunks per row of the wave tile
        constexpr int RPI = 64 / CPRW;         // rows per store instruction
        // Nontemporal stores: C does not stay dirty in the XCDs' L2s, whose
        // write-back at the end of the kernel otherwise delays the next
        // launch (4096^3: 3.0 -> 1.4 us between back-to-back launches, the
        // stores themselves ~1 us slower, overlapped with other workgroups)
#pragma unroll
        for (int it = 0; it < WTM / RPI; ++it) {
            const int m = it * RPI + lane / CPRW, c = lane % CPRW;
            const u32x4 v = *reinterpret_cast<const lds_u32x4*>((size_t)(wbase + m * PITCH + c * 16));
            const int gm = wrow0 + m, gn = wcol0 + 8 * c;
            if (gm < M && gn < N) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + (int64_t)gm * N + gn));
        }
        ts_end();
        return;
    }
    // ---- epilogue with beta: read-modify-write straight from the accumulators.
    // Half the wave tile's C at a time is loaded (clamped addresses) before
    // any of it is stored: a load issued after a store to C waits for it, one
    // round trip per 4 columns otherwise ----
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        u32x2 old[FM / 2][FN];
#pragma unroll
        for (int jj = 0; jj < FM / 2; ++jj) {
            const int gm = min(wrow0 + 16 * (half * FM / 2 + jj) + q, M - 1);
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int gn = min(wcol0 + 16 * i + 4 * h, N - 4);
                old[jj][i] = *reinterpret_cast<const u32x2*>(C + (int64_t)gm * N + gn);
            }
        }
#pragma unroll
        for (int jj = 0; jj < FM / 2; ++jj) {
            const int j = half * FM / 2 + jj;
            const int gm = wrow0 + 16 * j + q;
            if (gm >= M) continue;
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int gn = wcol0 + 16 * i + 4 * h;
                if (gn >= N) continue;
                const f32x4 v = acc[8 * i + j];
                const u32x2 c = old[jj][i];
                const float r0 = fmaf(p.beta, h2f(c.x & 0xffffu), p.alpha * v[0]);
                const float r1 = fmaf(p.beta, h2f(c.x >> 16), p.alpha * v[1]);
                const float r2 = fmaf(p.beta, h2f(c.y & 0xffffu), p.alpha * v[2]);
                const float r3 = fmaf(p.beta, h2f(c.y >> 16), p.alpha * v[3]);
                *reinterpret_cast<u32x2*>(C + (int64_t)gm * N + gn) = u32x2{pack2h(r0, r1), pack2h(r2, r3)};
            }
        }
    }
    ts_end();
}

// (a template so that every translation unit that includes this header can
// see it without defining the kernel twice; launched as gemm_f16_big<Big>)
template <class CF>
__global__ void __launch_bounds__(CF::NT) gemm_f16_big(Args p) {
    big_body<CF, false>(p, nullptr);
}

// the K split (Args: nsplit, ktps, part, counters)
template <class CF>
__global__ void __launch_bounds__(CF::NT) gemm_f16_big_split(Args p) {
    big_body<CF, false, true>(p, nullptr);
}

// the same kernel with the phase timestamps (ts: kTsWords words per workgroup)
template <class CF>
__global__ void __launch_bounds__(CF::NT) gemm_f16_big_ts(Args p, unsigned long long* ts) {
    big_body<CF, true>(p, ts);
}

}  // namespace dma
}  // namespace clove
