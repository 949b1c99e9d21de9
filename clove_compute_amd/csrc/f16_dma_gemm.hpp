// FP16 GEMM for large, aligned shapes on gfx950.
//
//   C[M,N] = alpha * A[M,K] @ B[K,N] + beta * C      fp32 accumulation
//
// Requirements (checked by the host): K % BK == 0, N % 8 == 0, M >= 1,
// N >= 8, A/B/C 16-byte aligned, each operand < 2^31 bytes.  Ragged M and N
// are handled by clamping the load rows/columns (their outputs are never
// stored).
//
// LDS holds both operands K-contiguous per row with the same XOR swizzle,
//   A stage: [BM rows m][BK k],  B stage: [BN rows n][BK k],
// 16-byte chunk c of row r at slot c ^ swz(r), so every MFMA fragment is one
// conflict-free ds_read_b128.  (An LDS read instruction costs the same issue
// time for 8 and 16 bytes per lane, so the transposing 8-byte reads
// ds_read_b64_tr_b16 would double the B read cost; LDS issue time is what
// bounds this kernel.)
//
// Staging.  A (K-contiguous in memory) goes global -> LDS by LDS DMA
// (buffer_load_dwordx4 ... lds): a wave instruction writes 64 consecutive
// 16-byte slots and each lane fetches the chunk that belongs in its slot.  B
// (N-contiguous) is loaded into VGPRs as 8 k-rows x 16 bytes per thread,
// transposed 8x8 with v_perm_b32 and written as 8 ds_write_b128.
//
// MFMA: v_mfma_f32_32x32x16_f16 with the B tile as the MFMA "A" operand
// (rows = n) and the A tile as the MFMA "B" operand (cols = m); a lane holds
// 8 consecutive k of one row for both.  Each wave owns WTM x WTN outputs.
//
// Pipeline.  LDS holds three A stages and two B stages (160 KB).  During K
// tile t the thread writes the transposed B of tile t+1 from VGPRs (spread
// over the first k-steps), then loads the B rows of tile t+2 into the same
// VGPRs and issues the A DMA of tile t+2.  The A DMA is inline asm with explicit vmcnt
// waits, since the compiler would otherwise wait for every DMA in flight
// before any LDS read.  One barrier per K tile, placed mid-way through the last
// k-step so that its second half hides the first fragment reads of the next
// tile.  MFMAs, fragment reads and memory instructions are interleaved in a
// fixed order (sched_barrier) that never queues more than one LDS write or
// memory instruction per MFMA.
//
// Epilogue (beta == 0): the wave's fp16 tile goes through LDS so that every
// global store is a full 16-byte lane of a contiguous row segment.
#pragma once

#include "common.hpp"

namespace clove {
namespace dma {

using namespace hw;

typedef short i16x4 __attribute__((ext_vector_type(4)));

struct Args {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    int M, N, K;
    float alpha, beta;
    int64_t sA, sB, sC;  // batch strides (elements)
    int tiles_m, tiles_n;
};

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int NW = WGM * WGN, NT = NW * 64;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int KSTEPS = BK / 16;
    static constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    static constexpr int DMA_A = A_ELEMS / 8 / NT;  // A DMA instructions per thread per K tile
    static constexpr int CPR = BK / 8;              // 16-byte chunks per LDS row
    static constexpr int A_STAGES = 3, B_STAGES = 2;
    static constexpr size_t LDS_BYTES = (size_t)(A_STAGES * A_ELEMS + B_STAGES * B_ELEMS) * 2;
    static_assert(LDS_BYTES <= 163840, "LDS");
    static_assert(NW * WTM * (WTN * 2 + 16) <= (int)LDS_BYTES, "epilogue staging");
    static_assert(BK == 64, "K tile (swizzle, 8-row B blocks)");
    static_assert(A_ELEMS % (8 * NT) == 0 && 64 % CPR == 0, "A DMA split");
    static_assert((BK / 8) * (BN / 8) == NT, "one 8x8 B block per thread");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && KSTEPS % 2 == 0, "wave tile");
    static_assert(FM * FN >= 2 * (FM + FN) && FM * FN % 2 == 0, "slots for reads and B writes");
};

template <int BK>
__device__ __forceinline__ int swz_a(int r) {
    if constexpr (BK == 64) return (r + (r >> 3)) & 7;
    else return ((r >> 1) + (r >> 3)) & 3;
}

// s_waitcnt with only the vector-memory counter constrained
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14);
}

// One 16-byte-per-lane LDS DMA: buffer_load_dwordx4 ... lds writes lane l's
// 16 bytes at LDS byte address m0 + 16 l.  Issued as inline asm so that the
// compiler does not treat it as a possible writer of the stage being read
// (it would otherwise wait for every DMA in flight before each LDS read);
// completion is tracked explicitly with vmcnt + a workgroup barrier.
__device__ __forceinline__ void dma16(const u32x4& rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
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

template <class CF>
__device__ __forceinline__ void tile_coords(const Args& p, int& batch, int& tm, int& tn) {
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    // workgroups are dealt to the 8 XCDs round-robin: give each XCD a
    // contiguous range of tiles so its L2 sees shared A and B panels
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int per_batch = p.tiles_m * p.tiles_n;
    batch = bid / per_batch;
    int tile = bid - batch * per_batch;
    constexpr int GM = 8;
    const int group = tile / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gm = min(p.tiles_m - first_m, GM);
    const int in_group = tile - group * GM * p.tiles_n;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

template <class CF>
__global__ void __launch_bounds__(CF::NT) gemm_f16_dma(Args p) {
    constexpr int BM = CF::BM, BN = CF::BN, BK = CF::BK, NW = CF::NW;
    constexpr int FM = CF::FM, FN = CF::FN, KSTEPS = CF::KSTEPS;
    constexpr int A_BYTES = CF::A_ELEMS * 2, B_BYTES = CF::B_ELEMS * 2;
    constexpr int NMF = FM * FN;    // MFMAs per k-step
    constexpr int NR = FM + FN;     // fragment reads per k-step
    __shared__ __attribute__((aligned(1024))) uint16_t smem[CF::LDS_BYTES / 2];

    int batch, tm, tn;
    tile_coords<CF>(p, batch, tm, tn);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / CF::WGN, wn = wave % CF::WGN;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;
    const int KT = K / BK;

    const u32x4 ra = make_rsrc(p.A + batch * p.sA, (unsigned)M * K * 2);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.B + batch * p.sB), (short)0, K * N * 2, 0x00020000);
    const unsigned lds_base = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) uint16_t*)smem));
    const unsigned lds_a = lds_base, lds_b = lds_base + CF::A_STAGES * A_BYTES;

    // Swizzle arithmetic.  For a row r = 32 x + (lane % 32) (x any integer)
    // swz(r) = (r + r/8) % 8 = (s0 + 4 x) % 8 = s0 ^ (4 (x % 2)), with
    // s0 = (lane % 8 + (lane / 8) % 4) % 8, so every fragment address is a
    // per-lane value plus a constant.
    static_assert(BM == 256 && BN == 256 && NW == 4 && CF::WTM == 128 && CF::WTN == 128,
                  "address arithmetic below is written for 256x256x64 with 2x2 waves");

    // ---- A: LDS DMA.  Instruction i of wave w fills rows 32 i + 8 w + lane/8,
    // slot lane % 8; rows >= M read as zero through the buffer range check ----
    const int dsw = ((lane >> 3) + wave) & 7;  // swz of the DMA row, for even i
    int offA[2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
        offA[e] = 2 * ((m0 + 8 * wave + (lane >> 3)) * K + 8 * ((lane & 7) ^ dsw ^ (4 * e)));
    auto dma_a = [&](int kt, int ast, int i) {
        dma16(ra, lds_a + ast * A_BYTES + (i * NW + wave) * 1024, offA[i & 1],
              kt * BK * 2 + i * 32 * K * 2);
    };

    // ---- B: thread owns k-rows 8kb..8kb+7 x columns 8cb..8cb+7 of the tile ----
    const int cb = tid % (BN / 8), kb = tid / (BN / 8);
    const int offB = 2 * (8 * kb * N + min(n0 + 8 * cb, N - 8));
    u32x4 breg[8];
    // compiler-visible loads: the compiler inserts the vmcnt wait before each
    // use (counting only these loads, so it may also wait for A DMAs issued in
    // between, which is safe)
    auto load_b = [&](int kt, int rr) {
        breg[rr] = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(rb, offB, (kt * BK + rr) * N * 2, 0));
    };
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    // column c of the 8x8 block: 8 k-values, two per dword, from the 8 loaded
    // rows, written to B^T row n = 8cb + c, chunk kb (swz(n) = (c + cb) % 8)
    auto write_b = [&](int bst, int c) {
        const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;
        const int d = c >> 1;
        const u32x4(&r)[8] = breg;
        u32x4 w;
        w.x = __builtin_amdgcn_perm(r[1][d], r[0][d], sel);
        w.y = __builtin_amdgcn_perm(r[3][d], r[2][d], sel);
        w.z = __builtin_amdgcn_perm(r[5][d], r[4][d], sel);
        w.w = __builtin_amdgcn_perm(r[7][d], r[6][d], sel);
        const unsigned off = (8 * cb + c) * BK * 2 + 16 * (kb ^ ((c + cb) & 7));
        *reinterpret_cast<lds_u32x4*>((size_t)(lds_b + bst * B_BYTES + off)) = w;
    };

    // ---- fragment reads: row 32 x + lane % 32 of the wave tile, chunk 2t + lane/32 ----
    const int s0 = ((lane & 7) + ((lane >> 3) & 3)) & 7;
    unsigned foff[KSTEPS][2];  // [t][x % 2]
#pragma unroll
    for (int t = 0; t < KSTEPS; ++t)
#pragma unroll
        for (int e = 0; e < 2; ++e)
            foff[t][e] = (lane & 31) * BK * 2 + 16 * (((2 * t + (lane >> 5)) ^ s0) ^ (4 * e));
    auto read_one = [&](int r, int ast, int bst, int t, f16x8 (&fa)[FM], f16x8 (&fb)[FN]) {
        if (r < FM) {
            const unsigned a = lds_a + ast * A_BYTES + wm * CF::WTM * BK * 2 + r * 32 * BK * 2 + foff[t][r & 1];
            fa[r] = bitcast<f16x8>(*reinterpret_cast<const lds_u32x4*>((size_t)a));
        } else {
            const int i = r - FM;
            const unsigned a = lds_b + bst * B_BYTES + wn * CF::WTN * BK * 2 + i * 32 * BK * 2 + foff[t][i & 1];
            fb[i] = bitcast<f16x8>(*reinterpret_cast<const lds_u32x4*>((size_t)a));
        }
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    auto mfma = [&](int n, const f16x8 (&fa)[FM], const f16x8 (&fb)[FN]) {
        const int i = n / FM, j = n % FM;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[i], fa[j], acc[i][j], 0, 0, 0);
    };

    // ---- prologue: B^T of tile 0 written, B rows of tile 1 in VGPRs, A tiles 0, 1 in flight ----
    // per K tile the issue order is: 8 B row loads, then the A DMA
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) load_b(0, rr);
#pragma unroll
    for (int i = 0; i < CF::DMA_A; ++i) dma_a(0, 0, i);
#pragma unroll
    for (int c = 0; c < 8; ++c) write_b(0, c);
    const int k1 = min(1, KT - 1);
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) load_b(k1, rr);
#pragma unroll
    for (int i = 0; i < CF::DMA_A; ++i) dma_a(k1, 1, i);
    stage_barrier<vmcnt_imm(8 + CF::DMA_A)>();  // A tile 0 (16 later ops) and B^T tile 0

    f16x8 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int r = 0; r < NR; ++r) read_one(r, 0, 0, 0, fa[0], fb[0]);

    int ast = 0;   // A stage of tile kt
    int bst = 0;   // B stage of tile kt
    // Slot plan over k-steps 0 .. KSTEPS-2 (slot g = NMF t + n; fragment
    // reads of k-step t+1 occupy n < NR of every k-step): the 8 transposed B
    // writes of tile kt+1 at g = 8..15, then (their registers read) the 8 B
    // row loads of tile kt+2 at g = 16..23 and its A DMA from g = 24.
    constexpr int NG = NMF * (KSTEPS - 1);
    static_assert(NMF == 16 && NR == 8 && NG >= 24 + CF::DMA_A, "slot plan");
#pragma unroll 1
    for (int kt = 0; kt < KT; ++kt) {
        const int ast1 = ast == 2 ? 0 : ast + 1;    // tile kt+1
        const int ast2 = ast1 == 2 ? 0 : ast1 + 1;  // tile kt+2 (read last during tile kt-1)
        const int bst1 = bst ^ 1;
        const int k2 = min(kt + 2, KT - 1);
#pragma unroll
        for (int t = 0; t < KSTEPS - 1; ++t) {
            const int cur = t & 1;
#pragma unroll
            for (int n = 0; n < NMF; ++n) {
                const int g = NMF * t + n;
                mfma(n, fa[cur], fb[cur]);
                if (n < NR) read_one(n, ast, bst, t + 1, fa[cur ^ 1], fb[cur ^ 1]);
                if (g >= 8 && g < 16) write_b(bst1, g - 8);
                if (g >= 16 && g < 24) load_b(k2, g - 16);
                if (g >= 24 && g - 24 < CF::DMA_A) dma_a(k2, ast2, g - 24);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        {
            constexpr int cur = (KSTEPS - 1) & 1;
#pragma unroll
            for (int n = 0; n < NMF / 2; ++n) {
                mfma(n, fa[cur], fb[cur]);
                __builtin_amdgcn_sched_barrier(0);
            }
            // A of tile kt+1 landed (the 8 + DMA_A ops of tile kt+2 may be in
            // flight), B^T of tile kt+1 written, stage of tile kt-1 free
            stage_barrier<vmcnt_imm(8 + CF::DMA_A)>();
#pragma unroll
            for (int n = NMF / 2; n < NMF; ++n) {
                mfma(n, fa[cur], fb[cur]);
                const int r = n - NMF / 2;
                if (r < NR) read_one(r, ast1, bst1, 0, fa[cur ^ 1], fb[cur ^ 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int r = NMF / 2; r < NR; ++r) read_one(r, ast1, bst1, 0, fa[cur ^ 1], fb[cur ^ 1]);
        }
        ast = ast1;
        bst = bst1;
    }
    // every load has landed and every wave is done with the stages
    stage_barrier<vmcnt_imm(0)>();

    uint16_t* C = p.C + batch * p.sC;
    const int wrow0 = m0 + wm * CF::WTM, wcol0 = n0 + wn * CF::WTN;
    if (p.beta == 0.0f) {
        // ---- epilogue through LDS: lane holds m = 32j + l%32, n = 32i + 8q + 4(l/32) + 0..3 ----
        constexpr int PITCH = CF::WTN * 2 + 16;  // bytes; the pad spreads rows over the banks
        const unsigned wbase = lds_base + wave * CF::WTM * PITCH;
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = 32 * j + (lane & 31), n = 32 * i + 8 * q + 4 * (lane >> 5);
                    const u32x2 v = {pack2h(p.alpha * acc[i][j][4 * q], p.alpha * acc[i][j][4 * q + 1]),
                                     pack2h(p.alpha * acc[i][j][4 * q + 2], p.alpha * acc[i][j][4 * q + 3])};
                    *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(
                        (size_t)(wbase + m * PITCH + n * 2)) = v;
                }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes are visible to its reads
        constexpr int CPRW = CF::WTN / 8;      // 16-byte chunks per row of the wave tile
        constexpr int RPI = 64 / CPRW;         // rows per store instruction
#pragma unroll
        for (int it = 0; it < CF::WTM / RPI; ++it) {
            const int m = it * RPI + lane / CPRW, c = lane % CPRW;
            const u32x4 v = *reinterpret_cast<const lds_u32x4*>((size_t)(wbase + m * PITCH + c * 16));
            const int gm = wrow0 + m, gn = wcol0 + 8 * c;
            if (gm < M && gn < N) *reinterpret_cast<u32x4*>(C + (int64_t)gm * N + gn) = v;
        }
        return;
    }
    // ---- epilogue with beta: read-modify-write straight from the accumulators ----
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int gm = wrow0 + 32 * j + (lane & 31);
        if (gm >= M) continue;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int gn = wcol0 + 32 * i + 8 * q + 4 * (lane >> 5);
                if (gn >= N) continue;
                float r0 = p.alpha * acc[i][j][4 * q], r1 = p.alpha * acc[i][j][4 * q + 1];
                float r2 = p.alpha * acc[i][j][4 * q + 2], r3 = p.alpha * acc[i][j][4 * q + 3];
                uint16_t* dst = C + (int64_t)gm * N + gn;
                const u32x2 c = *reinterpret_cast<const u32x2*>(dst);
                r0 = fmaf(p.beta, h2f(c.x & 0xffffu), r0);
                r1 = fmaf(p.beta, h2f(c.x >> 16), r1);
                r2 = fmaf(p.beta, h2f(c.y & 0xffffu), r2);
                r3 = fmaf(p.beta, h2f(c.y >> 16), r3);
                *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(r0, r1), pack2h(r2, r3)};
            }
        }
    }
}

}  // namespace dma
}  // namespace clove
