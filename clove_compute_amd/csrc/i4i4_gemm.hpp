// Group-wise INT4 x INT4 GEMM on int8 MFMA for gfx950: gemm_int4's prefill
// shapes (N >= 64 activation columns).
//
//   C[m, n] = sum_g sA[m,g] * sB[g,n] * P_g[m,n]
//   P_g     = sum_{k in g} (qA[m,k] - zA[m,g]) * (qB[k,n] - zB[g,n])     (int32, exact)
//
// Both factors of every product are small integers: with zero points in
// [-112, 127] and nibbles in [0, 15], q - z lies in [-127, 127] and is an exact
// int8, so v_mfma_i32_32x32x32_i8 forms P_g exactly (|P_g| <= 128 * 127^2 <
// 2^31) at twice the fp16 MFMA rate, and each group is folded into an fp32
// accumulator with its scale: acc = fma(sA * sB, float(P_g), acc), the
// oracle's group-wise arithmetic.  A zero point outside that range makes the
// scale NaN, so the outputs it touches are NaN rather than silently wrong.
//
// Operands.
//   A   [M, K/2] packed weight rows (even k in the high nibble), streamed once
//       from HBM by LDS DMA in 128-byte row pieces (two groups per stage)
//   Bt  [G, Npad, 128] int8 qB - zB, group-major: the 128 columns of one group
//       and column tile are 16 contiguous KB.  Within every 8 k the bytes are
//       in the order k0 k2 k4 k6 k1 k3 k5 k7, the order in which a packed
//       weight dword unpacks (high nibbles, then low nibbles), so the weight
//       side needs no byte permute.  Written by i4_prep_bt once per call (the
//       activations are small next to the weights) with the fp32 scales
//       sBf [G, Npad]
//   zA, sA [M, G] fp16, gathered per stage as the dword holding groups (g, g+1)
//
// Tiles.  A workgroup of 8 waves owns 64 weight rows x 128 columns.  Waves
// 0-3 (set 0) take the even group of each two-group stage and waves 4-7
// (set 1) the odd one; within a set a wave owns 32 rows x 64 columns (two
// 32x32 blocks), so the two waves of a row pair unpack the same rows.  The
// weight fragment is the MFMA "A" operand (a lane unpacks one weight row with
// its zero point) and the Bt fragment "B", so a lane's outputs are one column
// 32 b + m per block and 16 rows.  In k-step s of a group, lane half h holds
// k = 64 h + 16 s .. +15 of both operands.  The unpack lane also turns its
// row's fp16 scale into fp32 (NaN for a bad zero point); with the lane's
// column scale sB it forms the group's scale products sA[row] * sB[col] for
// all the wave's outputs as one v_mfma_f32_32x32x2_f32 outer product per
// column block (the unpack lane is the A operand's row, the column lane the B
// operand's column; k = 1 carries zeros), which lands in the accumulator
// layout: the fold is then 2 VALU per output (convert, fma) and no scale
// crosses lanes.  The int32 sums and scale products are double-buffered: a
// group's MFMAs run interleaved with the fold of the wave's previous group,
// so the fold (VALU) overlaps the matrix core.
//
// Streams.  The weight rows come from HBM, Bt from L2.  Vector-memory
// completions count in issue order per wave, so the two streams are issued
// by different waves: set 0 issues the weight pieces (and zA / sA), set 1 the
// Bt pieces (and sBf), each LA - 1 (LB - 1) stages ahead from an LA (LB) deep
// ring, and each wave waits only for its own stream before the workgroup
// barrier that publishes a stage.  One stage ahead is enough: a stage's loads
// land within the stage of compute they overlap (~1.5 us), and deeper rings
// only make every workgroup's first stage wait behind the whole chip's
// initial burst (per-workgroup timestamps at 4096x11008 N = 128: first stage
// after 6.1 us with 5 + 2 stages in flight, after 2.6 us with 1 + 1; the
// steady-state stage time the same).
//
// Partials mode (PART, the group-partials test hook): each wave stores its
// group's int32 sums P_g to P [M, N, G] instead of folding them (INT32_MIN
// where the row's or the column's zero point is outside the exact range), and
// there is no end phase.
//
// End.  Set 1 hands its fp32 sums to set 0 through LDS (fixed order).
// Split-K over groups when the tiles do not cover the CUs: fp32 partial tiles,
// the last workgroup to arrive sums them in split order (deterministic).  The
// output tile goes through LDS so that every store is 16 contiguous bytes.
//
// LDS (16-byte chunks XOR-swizzled so every fragment read is conflict free:
// a 16-byte read serves 16 lanes per clock from 256 bytes of banks, i.e. two
// 128-byte rows, and 16 consecutive rows r reading chunk c hit the 16
// distinct slots (r & 1, c ^ ((r >> 1) & 7)) of that window):
//   weight stage  64 rows x 128 B (chunk c of row r at slot c ^ ((r >> 1) & 7)),
//                 then the 64 (g, g+1) dwords of zA and of sA
//   Bt stage      2 groups x 128 columns x 128 B (chunk c of column n at
//                 slot c ^ ((n >> 1) & 7)), then 2 x 128 fp32 sBf
// Every weight wave issues DA DMAs per stage and every Bt wave DB (waves
// without a scale piece load a dummy into a junk slot), so the vmcnt waits
// count the same for every wave of a stream.
#pragma once

#include "common.hpp"
#include "f16_dma_gemm.hpp"

namespace clove {
namespace i4i4 {

using namespace hw;
using dma::make_rsrc;
using dma::vmcnt_imm;

struct Args {
    const uint8_t* A;     // [M, K/2]
    const uint16_t* sA;   // [M, G] fp16
    const uint16_t* zA;   // [M, G] fp16
    const int8_t* Bt;     // [G, Npad, 128] int8, qB - zB (i4_prep_bt)
    const float* sBf;     // [G, Npad] fp32, NaN where zB is out of range (i4_prep_bt)
    uint16_t* C;          // [M, N] fp16
    int M, N, K, G, Npad;
    int tiles_m, tiles_n, nsplit, gps;  // gps: groups per split, even (G is even)
    int vec_store;        // 16-byte output stores (N % 8 == 0, C 16-byte aligned)
    float* part;
    unsigned* counters;
    int* P;               // partials mode: [M, N, G] int32
};

constexpr int NW = 8, NT = 512;
constexpr int BR = 64, BC = 128;
constexpr int NB = 2;          // 32x32 blocks per wave: 32 rows x 64 columns
constexpr int LA = 2, LB = 2;  // weight / Bt stages in the rings (one stage ahead, see the header)
constexpr int DA = 3, DB = 9;  // DMAs per stage of a weight wave / of a Bt wave
constexpr int ZA_OFF = BR * 128, SA_OFF = ZA_OFF + BR * 4, AST = SA_OFF + BR * 4;
constexpr int SB_OFF = 2 * BC * 128, BST = SB_OFF + 2 * BC * 4;
constexpr int BT0 = LA * AST;
constexpr int JUNK = BT0 + LB * BST;  // dummy DMA target, 1 KB
constexpr int LDS = JUNK + 1024;
constexpr int PREP_COLS = 64;         // i4_prep_bt columns per workgroup
static_assert(AST % 256 == 0 && BST % 256 == 0, "stage alignment");
static_assert(BR / 8 == 2 * 4 && 2 * BC * 128 / 1024 == 8 * 4, "DMA blocks per wave");
static_assert(LDS <= 160 * 1024, "LDS");
static_assert(BR * (BC + 8) * 2 <= BT0 + LB * BST && 4 * 64 * NB * 16 * 4 <= BT0 + LB * BST, "epilogue staging");
static_assert((LA - 2) * DA <= 63 && (LB - 2) * DB <= 63, "vmcnt range");

// The LDS DMAs of this kernel.  Their asm starts with five wait states: a
// VMEM instruction that reads an SGPR needs five after a VALU write of it, and
// the compiler, which does not see the load inside the asm, restores SGPRs it
// has spilled to VGPR lanes (v_readlane_b32) right in front of the asm (it does
// in the partials instantiation, whose SGPRs run out).  Without them the load
// can read a stale resource word: observed as weight rows read as zeros, and a
// memory fault.  Five wait states also cover the one after the M0 write.
__device__ __forceinline__ void dma16(const u32x4& rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
                 : "memory");
}
__device__ __forceinline__ void dma4(const u32x4& rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
                 : "memory");
}

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) unsigned lds_u32;
typedef __attribute__((address_space(3))) float lds_f32;

__device__ __forceinline__ u32x4 ld16(unsigned a) { return *reinterpret_cast<const lds_u32x4*>((size_t)a); }
__device__ __forceinline__ unsigned ld4(unsigned a) { return *reinterpret_cast<const lds_u32*>((size_t)a); }

// the LDS slot swizzle of a 128-byte row or column piece
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// fp16 zero point -> (ok, integer): nearest with ties to even, in [-112, 127]
__device__ __forceinline__ bool zero_ok(uint16_t h, int& z) {
    const float zf = rintf(h2f(h));
    const bool ok = zf >= -112.0f && zf <= 127.0f;
    z = ok ? (int)zf : 0;
    return ok;
}

// this wave's DMAs up to the last `r` stages of D each have landed
template <int D>
__device__ __forceinline__ void wait_stages(int r) {
    switch (r) {
        case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(D)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * D < 63 ? 2 * D : 63)); break;
        case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * D < 63 ? 3 * D : 63)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * D < 63 ? 4 * D : 63)); break;
    }
}

// LDS reads returned, then the workgroup barrier; the empty asm statements
// keep the compiler from moving LDS accesses across it
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Bt[g][n][k'] = int8(qB[k][n] - zB[g][n]) for n < N (0 for N <= n < Npad),
// k' the unpack order of every 8 k (k0 k2 k4 k6 k1 k3 k5 k7), and
// sBf[g][n] = sB[g][n] (0 past N, or for a null sB; NaN where zB is outside
// [-112, 127]).
// Grid (G, Npad / 64), 128 threads: the group's 128 packed rows of the
// 64-column slab are staged in LDS with coalesced loads, then thread (p, kq)
// writes columns 2p, 2p + 1 for k = 32 kq .. 32 kq + 31.
__global__ void __launch_bounds__(128) i4_prep_bt(const uint8_t* B, int ldb, const uint16_t* sB,
                                                  const uint16_t* zB, int N, int K, int Npad, int8_t* Bt,
                                                  float* sBf) {
    __shared__ __attribute__((aligned(16))) uint8_t rows[128][PREP_COLS / 2 + 4];
    const int g = blockIdx.x, tid = threadIdx.x;
    const int nb0 = blockIdx.y * (PREP_COLS / 2);  // first packed byte of the slab
    const int p = tid & 31, kq = tid >> 5;
    // the zero points and scales of this thread's two columns, loaded first so
    // that their latency overlaps the staging
    uint16_t zh[2] = {0, 0}, sh[2] = {0, 0};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int n = 2 * (nb0 + p) + c;
        if (n < N) {
            zh[c] = zB[(int64_t)g * N + n];
            sh[c] = sB ? sB[(int64_t)g * N + n] : (uint16_t)0;
        }
    }
    // stage: thread t loads 32 bytes of row t (bytes past the row end: 0)
    {
        const int k = g * 128 + tid;
        const uint8_t* src = B + (int64_t)k * ldb + nb0;
        const int avail = min(PREP_COLS / 2, ldb - nb0);
        unsigned w[8];
        if (k < K && avail == PREP_COLS / 2 && ((reinterpret_cast<uintptr_t>(src) & 3) == 0)) {
#pragma unroll
            for (int d = 0; d < 8; ++d) w[d] = reinterpret_cast<const unsigned*>(src)[d];
        } else {
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                unsigned v = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (k < K && 4 * d + e < avail) v |= (unsigned)src[4 * d + e] << (8 * e);
                w[d] = v;
            }
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) *reinterpret_cast<unsigned*>(&rows[tid][4 * d]) = w[d];
    }
    __syncthreads();
    int z[2];
    bool in[2];
    float s[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int n = 2 * (nb0 + p) + c;
        in[c] = n < N;
        z[c] = 0;
        s[c] = 0.0f;
        if (in[c]) {
            const bool ok = zero_ok(zh[c], z[c]);
            s[c] = ok ? h2f(sh[c]) : __builtin_nanf("");
        }
    }
    // column 2p is the high nibble of byte p, column 2p + 1 the low one
    unsigned o[2][8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // 8-k chunk j of this thread's 32 k
        unsigned b8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b8[e] = rows[32 * kq + 8 * j + e][p];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            unsigned v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int q = c == 0 ? (int)(b8[e] >> 4) : (int)(b8[e] & 15u);
                v[e] = in[c] ? (unsigned)(q - z[c]) & 0xffu : 0u;
            }
            o[c][2 * j] = v[0] | (v[2] << 8) | (v[4] << 16) | (v[6] << 24);
            o[c][2 * j + 1] = v[1] | (v[3] << 8) | (v[5] << 16) | (v[7] << 24);
        }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int n = 2 * (nb0 + p) + c;
        u32x4* dst = reinterpret_cast<u32x4*>(Bt + ((int64_t)g * Npad + n) * 128 + 32 * kq);
        dst[0] = u32x4{o[c][0], o[c][1], o[c][2], o[c][3]};
        dst[1] = u32x4{o[c][4], o[c][5], o[c][6], o[c][7]};
        if (kq == 0) sBf[(int64_t)g * Npad + n] = s[c];
    }
}

template <bool PART>
__global__ void __launch_bounds__(NT) i4i4_gemm(Args p) {
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int set = wave >> 2, rw = wave & 1, cw = (wave >> 1) & 1;

    // ---- tile, split, group range (split-major: workgroups in flight
    // together share their groups of Bt) ----
    const int ntiles = p.tiles_m * p.tiles_n;
    const int split = blockIdx.x / ntiles;
    const int tile = blockIdx.x - split * ntiles;
    const int tn = tile % p.tiles_n, tm = tile / p.tiles_n;
    const int m0 = tm * BR, n0 = tn * BC;
    const int M = p.M, K = p.K, G = p.G, Npad = p.Npad;
    const int gbeg = split * p.gps;
    const int gend = min(G, gbeg + p.gps);
    const int nst = (gend - gbeg) >> 1;  // two groups per stage

    const unsigned lds0 = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) unsigned char*)smem));
    const int KB = K >> 1;  // bytes per weight row
    const u32x4 ra = make_rsrc(p.A, (unsigned)M * KB);
    const u32x4 rb = make_rsrc(p.Bt, (unsigned)G * Npad * 128);
    const u32x4 rs = make_rsrc(p.sBf, (unsigned)G * Npad * 4);
    const u32x4 rza = make_rsrc(p.zA, (unsigned)M * G * 2);
    const u32x4 rsa = make_rsrc(p.sA, (unsigned)M * G * 2);

    // ---- per-lane DMA offsets (the stage's first group is the soffset) ----
    // weight waves: blocks 2 wave + i = rows 8 j .. 8 j + 7 (1 KB); wave 0 zA,
    //   wave 1 sA, waves 2-3 a dummy dword
    // Bt waves: blocks j = 8 (wave - 4) + i = group j >> 4 (one wave-uniform
    //   group per wave), columns 8 (j & 15) .. 8 (j & 15) + 7; wave 4 the
    //   scales of both groups, waves 5-7 a dummy piece
    int off[8];
    int offm = 0;
    if (set == 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = 8 * (2 * wave + i) + (lane >> 3);
            off[i] = (m0 + r) * KB + 16 * ((lane & 7) ^ swz(r));
        }
        if (wave < 2) offm = 2 * ((m0 + lane) * G);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = 8 * ((8 * (wave - 4) + i) & 15) + (lane >> 3);
            off[i] = (n0 + n) * 128 + 16 * ((lane & 7) ^ swz(n));
        }
        if (wave == 4) offm = 4 * ((lane >> 5) * Npad + n0 + 4 * (lane & 31));
    }
    auto issue_a = [&](int t) {
        const int gs = gbeg + 2 * t;
        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)((t % LA) * AST));
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16(ra, st + (2 * wave + i) * 1024, off[i], gs * 64);
        if (wave == 0) dma4(rza, st + ZA_OFF, offm, gs * 2);
        else if (wave == 1) dma4(rsa, st + SA_OFF, offm, gs * 2);
        else dma4(rsa, lds0 + JUNK + 256 * (wave - 2), 0, 0);
    };
    auto issue_b = [&](int t) {
        const int gs = gbeg + 2 * t;
        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(BT0 + (t % LB) * BST));
        const int soff = (gs + ((wave - 4) >> 1)) * Npad * 128;
#pragma unroll
        for (int i = 0; i < 8; ++i) dma16(rb, st + (8 * (wave - 4) + i) * 1024, off[i], soff);
        if (wave == 4) dma16(rs, st + SB_OFF, offm, gs * Npad * 4);
        else dma16(rs, lds0 + JUNK, 0, 0);
    };

    // ---- fragment addressing: lane (m, h); its weight row rA unpacks, its
    // outputs are rows 32 rw + 8 j + 4 h + e and columns 64 cw + 32 b + m ----
    const int m = lane & 31, h = lane >> 5;
    const int rA = 32 * rw + m;
    const unsigned aoff0 = rA * 128 + 16 * ((4 * set + 2 * h) ^ swz(rA));
    const unsigned aoff1 = rA * 128 + 16 * ((4 * set + 2 * h + 1) ^ swz(rA));
    const int ncol0 = 64 * cw;
    const unsigned bbase = set * (BC * 128);
    const unsigned sbase = SB_OFF + set * (BC * 4) + 4 * (ncol0 + m);
    const int half = 16 * set;  // the fp16 half of a (g, g+1) dword that is this wave's group

    f32x16 facc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) facc[b][v] = 0.0f;

    // one group: wait for its stage, refill the ring, MFMAs into `cur` with
    // the fold of `prev` (the previous group's sums and scales) interleaved
    auto step = [&](int t, i32x16 (&cur)[NB], f32x16 (&spc)[NB], const i32x16 (&prev)[NB],
                    const f32x16 (&spp)[NB]) {
        const int rem = nst - 1 - t;
        if (set == 0) wait_stages<DA>(min(rem, LA - 2));
        else wait_stages<DB>(min(rem, LB - 2));
        lds_barrier();
        if (set == 0) {
            if (t + LA - 1 < nst) issue_a(t + LA - 1);
        } else {
            if (t + LB - 1 < nst) issue_b(t + LB - 1);
        }
        const unsigned sa_st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)((t % LA) * AST));
        const unsigned sb_st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(BT0 + (t % LB) * BST));

        // ---- the LDS reads of the group's operands, issued together ----
        const unsigned zw = ld4(sa_st + ZA_OFF + 4 * rA);
        const unsigned sw = ld4(sa_st + SA_OFF + 4 * rA);
        const u32x4 p0 = ld16(sa_st + aoff0), p1 = ld16(sa_st + aoff1);
        float bcol[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            bcol[b] = *reinterpret_cast<const lds_f32*>((size_t)(sb_st + sbase + 4 * 32 * b));
        i32x4 bf[NB][4];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int n = ncol0 + 32 * b + m;
                bf[b][s] = bitcast<i32x4>(ld16(sb_st + bbase + n * 128 + 16 * ((4 * h + s) ^ swz(n))));
            }
        __builtin_amdgcn_sched_barrier(0);

        // ---- the unpack row: its weights as int8 q - z, and its scale (NaN
        // for a bad zero point); the scale products of the group's outputs
        // sA[row] * sB[col] as one 32x32x2 fp32 MFMA outer product per column
        // block (k = 0 carries the scales, k = 1 zeros), in the accumulator
        // layout, so the fold needs no row-scale exchange between lanes ----
        int z;
        const bool zok = zero_ok((uint16_t)(zw >> half), z);
        const float sa_row = zok ? (PART ? 0.0f : h2f((uint16_t)(sw >> half))) : __builtin_nanf("");
        const unsigned zp = (unsigned)(128 - z) * 0x01010101u;
        i32x4 wq[4];
        {
            const unsigned pk[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const unsigned hi = (pk[d] >> 4) & 0x0f0f0f0fu, lo = pk[d] & 0x0f0f0f0fu;
                wq[d >> 1][2 * (d & 1)] = (int)((hi + zp) ^ 0x80808080u);
                wq[d >> 1][2 * (d & 1) + 1] = (int)((lo + zp) ^ 0x80808080u);
            }
        }
        const float sa_op = h == 0 ? sa_row : 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b)
            spc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(sa_op, h == 0 ? bcol[b] : 0.0f, f32x16{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);

        // ---- NB x 4 MFMAs (k-step s of the column blocks; the next two
        // steps' Bt fragments read meanwhile) with the previous group's fold
        // (2 VALU per output: convert, fma; 8 per MFMA) placed between them.
        // The empty asm statements fence the fold into this region: its
        // inputs are defined at the start, its results used at the end
        // (otherwise the compiler sinks it to the next group's block, in
        // series with those MFMAs) ----
        if constexpr (PART) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s < 2) {
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const int n = ncol0 + 32 * b + m;
                        bf[b][s + 2] =
                            bitcast<i32x4>(ld16(sb_st + bbase + n * 128 + 16 * ((4 * h + s + 2) ^ swz(n))));
                    }
                }
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    cur[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wq[s], bf[b][s], s == 0 ? i32x16{} : cur[b],
                                                                   0, 0, 0);
            }
            // P[row][col][g]; a NaN row scale (the unpack lane's bad zero
            // point) or column scale (i4_prep_bt's) makes the product NaN and
            // marks the sum invalid
            const int g = gbeg + 2 * t + set;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int col = n0 + ncol0 + 32 * b + m;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = m0 + 32 * rw + 8 * (i >> 2) + 4 * h + (i & 3);
                    const float chk = spc[b][i];
                    if (row < M && col < p.N)
                        p.P[((int64_t)row * p.N + col) * G + g] = chk == chk ? cur[b][i] : (int)0x80000000u;
                }
            }
            return;
        }
        i32x16 pv[NB];
        f32x16 fa[NB], sp[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            pv[b] = prev[b];
            fa[b] = facc[b];
            sp[b] = spp[b];
            asm volatile("" : "+v"(pv[b]), "+v"(fa[b]), "+v"(sp[b]));
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < 2) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int n = ncol0 + 32 * b + m;
                    bf[b][s + 2] =
                        bitcast<i32x4>(ld16(sb_st + bbase + n * 128 + 16 * ((4 * h + s + 2) ^ swz(n))));
                }
            }
#pragma unroll
            for (int b = 0; b < NB; ++b)
                cur[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wq[s], bf[b][s], s == 0 ? i32x16{} : cur[b], 0, 0,
                                                               0);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) fa[b][i] = fmaf(sp[b][i], (float)pv[b][i], fa[b][i]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < 2) __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);  // DS reads
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            asm volatile("" : "+v"(fa[b]));
            facc[b] = fa[b];
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- prologue: each stream fills its ring ----
    if (set == 0) {
#pragma unroll
        for (int t = 0; t < LA - 1; ++t)
            if (t < nst) issue_a(t);
    } else {
#pragma unroll
        for (int t = 0; t < LB - 1; ++t)
            if (t < nst) issue_b(t);
    }

    // two sets of sums and scale products, alternating (no copies between
    // steps); the first fold reads zeros
    i32x16 ix[NB], iy[NB];
    f32x16 px[NB], py[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        iy[b] = i32x16{};
        py[b] = f32x16{};
    }
    int t = 0;
    for (; t + 1 < nst; t += 2) {
        step(t, ix, px, iy, py);
        step(t + 1, iy, py, ix, px);
    }
    // the last group's fold
    auto fold = [&](const i32x16 (&c)[NB], const f32x16 (&sp)[NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) facc[b][i] = fmaf(sp[b][i], (float)c[b][i], facc[b][i]);
    };
    if (t < nst) {
        step(t, ix, px, iy, py);
        fold(ix, px);
    } else {
        fold(iy, py);
    }
    // every DMA has landed and every wave is done with the stages
    dma::stage_barrier<vmcnt_imm(0)>();
    if constexpr (PART) return;

    // ---- set 1 hands its sums to set 0 (LDS, fixed order) ----
    {
        const unsigned xb = lds0 + (unsigned)((wave & 3) * 64 * NB * 16 * 4);
        if (set == 1) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    *reinterpret_cast<lds_f32*>((size_t)(xb + 4 * ((16 * b + v) * 64 + lane))) = facc[b][v];
        }
        __syncthreads();
        if (set == 0) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    facc[b][v] += *reinterpret_cast<const lds_f32*>((size_t)(xb + 4 * ((16 * b + v) * 64 + lane)));
        }
        __syncthreads();  // (the epilogue reuses this LDS)
    }

    // ---- split-K: fp32 partial tiles, the last workgroup to arrive sums them ----
    if (p.nsplit > 1) {
        constexpr int NC = 4 * NB;
        f32x4 v[NC];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[4 * b + q] = f32x4{facc[b][4 * q], facc[b][4 * q + 1], facc[b][4 * q + 2], facc[b][4 * q + 3]};
        float* slabs = p.part + (size_t)tile * p.nsplit * NC * 256 * 4;
        if (set == 0) splitk_publish<NC, 256>(slabs + (size_t)split * NC * 256 * 4, tid, v);
        if (!splitk_arrive_is_last(p.counters + tile, (unsigned)p.nsplit, reinterpret_cast<int*>(smem)))
            return;
        if (set == 0) splitk_reduce<NC, 256, false>(slabs, p.nsplit, split, tid, v);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) facc[b][4 * q + e] = v[4 * b + q][e];
    }

    // ---- epilogue: the fp16 tile through LDS (set 0 writes it), then 16-byte
    // row stores by all waves ----
    constexpr int PITCH = BC + 8;  // halves per LDS row (the pad spreads rows over the banks)
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
    if (set == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = 32 * rw + 8 * (i >> 2) + 4 * h + (i & 3);
                *reinterpret_cast<lds_u16*>((size_t)(lds0 + 2 * (row * PITCH + ncol0 + 32 * b + m))) =
                    f2h(facc[b][i]);
            }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < BR * BC / 8 / NT; ++c) {
        const int chunk = tid + NT * c;
        const int row = chunk >> 4, cc = chunk & 15;
        const int gm = m0 + row, gn = n0 + 8 * cc;
        if (gm >= M) continue;
        const u32x4 v = ld16(lds0 + 2 * (row * PITCH + 8 * cc));
        uint16_t* dst = p.C + (int64_t)gm * p.N + gn;
        if (p.vec_store && gn + 7 < p.N) {
            *reinterpret_cast<u32x4*>(dst) = v;
        } else {
            const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (gn + e < p.N) dst[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

}  // namespace i4i4
}  // namespace clove
