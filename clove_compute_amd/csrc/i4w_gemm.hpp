// MFMA GEMM with packed INT4 weight rows for gfx950: the prefill shapes of the
// W4A16 linear layer (T > 4 tokens) and of group-wise INT4 (N > 8 columns).
//
//   out[r, c] = sum_g  sw[r,g] * sx[g,c] * P_g[r,c]
//   P_g[r,c]  = sum_{k in group g} (q[r,k] - zw[r,g]) * x[c,k]
//
//   W  [R, K/2]  packed INT4 rows, even k in the high nibble (gemm_int4's A,
//                W4A16's weight), fp16 group scales sw and zero points zw [R, G]
//   X  [C, K]    fp16, K-contiguous: W4A16's activations, or for INT4 the
//                exact integers qB - zB of B transposed (prepared by i4w_prep_b)
//   sx [G, ldxs] fp32 per-(group, column) scale of X (INT4; absent for W4A16)
//
// q - z is exact in fp16 and so is every product with an fp16 x, so P_g is an
// fp32 MFMA sum of exact products (exact integers for INT4), and each group is
// folded into the fp32 accumulator with its scale: acc = fma(sw * sx, P_g, acc),
// the arithmetic of the reference-derived group-wise definition.
//
// Nibble unpack (10 VALU ops per 8 weights).  A dword w of packed weights holds
// k0..k7; hr = w & 0xf0f0f0f0 and lo = w & 0x0f0f0f0f, then one v_perm_b32 per
// byte b builds the half2 {hr.b, lo.b} with zero high bytes: the fp16
// subnormals 16 h * 2^-24 and l * 2^-24 (h, l the two nibbles).  One
// v_pk_fma_f16 by {2^11, 2^15} plus {-z 2^-9, -z 2^-9} gives (h - z) 2^-9 and
// (l - z) 2^-9, both exact; the 2^-9 is returned through the group scale
// (sw * 2^9, exact).
//
// Tiles.  A workgroup of NW = WR x WC waves owns BR = 32 FW WR weight rows by
// BC = 32 FX WC X rows; each wave owns (32 FW) x (32 FX) outputs as FW x FX
// v_mfma_f32_32x32x16_f16 tiles with the X fragment as the MFMA "A" operand
// and the weight fragment as "B", so a lane holds one weight row r (its scale
// and zero are per-lane scalars) and 16 X rows.  K advances one 128-wide group
// per stage.  Split-K over groups when the tiles do not cover the CUs: fp32
// partial tiles in scratch, the last-arriving workgroup of a tile sums them in
// split order (deterministic).
//
// Staging.  Everything a stage needs arrives by LDS DMA (inline asm, so that
// the compiler does not wait for all DMAs before each LDS read; completion is
// tracked with explicit vmcnt waits and one barrier per stage):
//   X   BC rows x 256 B, 16-byte chunk c of row x at slot c ^ (x & 15)
//   W   BR rows x 64 B,  chunk c of row r at slot c ^ ((r >> 2) & 3)
//   SC  BR dwords, the aligned dword holding sw[r, g]   (half chosen by parity)
//   ZR  BR dwords, the same for zw[r, g]
//   XS  64 NW fp32 of sx[g, c0 ...]                     (INT4 only)
// so X fragment reads (ds_read_b128) and weight reads (2 x ds_read_b128 per
// lane per group: 64 k of its row) are bank-conflict free.  Lane (r, h) of a
// weight tile covers k = 64 h .. 64 h + 63 of the group and uses dword s of it
// in k-step s; the X fragment of step s is x[c][64 h + 8 s .. + 7].
#pragma once

#include "common.hpp"
#include "f16_dma_gemm.hpp"

namespace clove {
namespace i4w {

using namespace hw;
using dma::dma16;
using dma::make_rsrc;
using dma::vmcnt_imm;

struct Args {
    const uint8_t* W;
    const uint16_t* wscale;  // [R, G] fp16
    const uint16_t* wzero;   // [R, G] fp16
    const uint16_t* X;       // [C, K] fp16 (rows >= C read as zero)
    const float* xs;         // [G, ldxs] fp32 or null
    uint16_t* out;           // OUT 0: [R, C] (C[m, n]),  OUT 1 / 2: [C, R] (Y[t, o] / H[t, o])
    int R, C, K, G, ldxs;    // OUT 2: R output rows, the weight has 2 R (gate, then up)
    float alpha, beta;       // OUT 1 epilogue: alpha * acc + beta * out
    int tiles_r, tiles_c, nsplit, gps;  // gps: groups per split
    float* part;
    unsigned* counters;
    // raw group-wise INT4 B for the streaming kernel's fused transpose
    // (i4w_stream.hpp): B [K, 8] bytes (N = 15 or 16), sB / zB [G, N] fp16
    const uint8_t* B;
    const uint16_t* bscale;
    const uint16_t* bzero;
    int N;
};

// KS: 16-wide k-steps per stage, 8 (a whole 128-k group) or 4 (half a group:
// smaller stages, so that two workgroups fit a CU's LDS and each SIMD can
// interleave two waves; the group is folded after its second stage)
template <int WR_, int WC_, int FW_, int FX_, int S_, int KS_ = 8>
struct Cfg {
    static constexpr int WR = WR_, WC = WC_, FW = FW_, FX = FX_, S = S_, KS = KS_;
    static constexpr int NW = WR * WC, NT = 64 * NW;
    static constexpr int BR = 32 * FW * WR, BC = 32 * FX * WC;
    static constexpr int SPG = 8 / KS;                  // stages per group
    static constexpr int XRB = 32 * KS, WRB = 8 * KS;   // bytes per X row / weight row per stage
    static constexpr int X_BYTES = BC * XRB, W_BYTES = BR * WRB, SC_BYTES = BR * 4;
    static constexpr int DX = X_BYTES / (1024 * NW);    // X DMA instructions per thread per stage
    static constexpr int DW = W_BYTES / (1024 * NW);    // weight DMA instructions
    static constexpr int DS = 2 * BR / (64 * NW);       // scale + zero DMA instructions
    static_assert(KS == 8 || KS == 4, "k-steps per stage");
    static_assert(NW == 2 || NW == 4 || NW == 8, "waves");
    static_assert(X_BYTES % (1024 * NW) == 0 && W_BYTES % (1024 * NW) == 0 && (2 * BR) % (64 * NW) == 0,
                  "DMA split");
    static_assert(BC <= 64 * NW, "one dword of sx per lane covers the tile");
    static_assert(S >= 2 && S <= 4, "stages");
    template <bool XS>
    static constexpr int stage_bytes() { return X_BYTES + W_BYTES + 2 * SC_BYTES + (XS ? 256 * NW : 0); }
    template <bool XS>
    static constexpr int lds_bytes() { return S * stage_bytes<XS>(); }
    template <bool XS>
    static constexpr int dma_per_stage() { return DX + DW + DS + (XS ? 1 : 0); }
};

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) unsigned lds_u32;

__device__ __forceinline__ u32x4 lds_read16(unsigned addr) {
    return *reinterpret_cast<const lds_u32x4*>((size_t)addr);
}
__device__ __forceinline__ unsigned lds_read4(unsigned addr) {
    return *reinterpret_cast<const lds_u32*>((size_t)addr);
}

// (the wait state after the M0 write, as in dma16)
__device__ __forceinline__ void dma4(const u32x4& rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
                 : "memory");
}

// (q - z) * 2^-9 for the 8 nibbles of one dword, in k order; zz = -z * 2^-9.
// Byte b holds k = 2b and 2b + 1: in the high and low nibble (the weights'
// packing), or with LO_FIRST in the low and high nibble (the order in which
// ds_read_b64_tr_b4 returns k rows)
template <bool LO_FIRST = false>
__device__ __forceinline__ f16x8 unpack8(unsigned w, f16x2 zz) {
    const unsigned hr = w & 0xf0f0f0f0u, lo = w & 0x0f0f0f0fu;
    const f16x2 mul = LO_FIRST ? f16x2{(_Float16)32768.0f, (_Float16)2048.0f}
                               : f16x2{(_Float16)2048.0f, (_Float16)32768.0f};
    f16x2 v[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const unsigned sel = LO_FIRST ? 0x0c000c00u | (unsigned)(4 + b) | ((unsigned)b << 16)
                                      : 0x0c000c00u | (unsigned)b | ((unsigned)(4 + b) << 16);
        const f16x2 sub = bitcast<f16x2>(__builtin_amdgcn_perm(lo, hr, sel));
        v[b] = __builtin_elementwise_fma(sub, mul, zz);
    }
    f16x8 r;
    r.s01 = v[0];
    r.s23 = v[1];
    r.s45 = v[2];
    r.s67 = v[3];
    return r;
}

// A 16-byte LDS read serves 16 lanes per clock from one 256-byte window of
// banks.  The 16 lanes of a fragment read take 16 consecutive rows, one chunk
// each, so the chunk is swizzled by the row bits above those that already
// separate rows within a window:
//   weight rows of 64 bytes (whole group: 4 rows per window) or 32 bytes
//   (half: 8 per window): chunk c at c ^ ((r >> 2) & 3) or c ^ ((r >> 3) & 1)
//   X rows of 256 bytes (one per window) or 128 bytes (two): chunk c at
//   c ^ (x & 15) or c ^ ((x >> 1) & 7)
// so rows r .. r + 15 reading one chunk hit 16 distinct 16-byte bank slots.
template <int KS>
__device__ __forceinline__ int swz_w(int r) {
    return KS == 8 ? ((r >> 2) & 3) : ((r >> 3) & 1);
}
template <int KS>
__device__ __forceinline__ int swz_x(int x) {
    return KS == 8 ? (x & 15) : ((x >> 1) & 7);
}

template <int IMM>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt(IMM);
}

template <class CF, bool XS, int OUT>
__global__ void __launch_bounds__(CF::NT) i4w_gemm(Args p) {
    constexpr int NW = CF::NW, FW = CF::FW, FX = CF::FX, S = CF::S;
    constexpr int BR = CF::BR, BC = CF::BC;
    constexpr int SB = CF::template stage_bytes<XS>();
    constexpr int OFF_W = CF::X_BYTES, OFF_SC = OFF_W + CF::W_BYTES, OFF_ZR = OFF_SC + CF::SC_BYTES,
                  OFF_XS = OFF_ZR + CF::SC_BYTES;
    constexpr int D = CF::template dma_per_stage<XS>();
    extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave % CF::WR, wc = wave / CF::WR;

    // ---- tile, split, K range.  Workgroups are dealt to the 8 XCDs round
    // robin (workgroup b runs on XCD b % 8) and each XCD has its own L2, so
    // the grid is renumbered to give every XCD a contiguous run of (tile,
    // split) pairs: the splits of a tile and the X-row tiles of a weight-row
    // tile then share one L2 (measured: split-K shapes 3-12 % faster) ----
    const int bid = gridDim.x % 8 == 0 ? (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8) : (int)blockIdx.x;
    const int split = bid % p.nsplit;
    const int tile = bid / p.nsplit;
    const int tc = tile % p.tiles_c, tr = tile / p.tiles_c;
    // OUT 2 (SwiGLU): in every 32-row block of the tile, rows 0..15 are the
    // gate rows of 16 outputs and rows 16..31 the up rows (weight rows R + o)
    // of the same outputs, so each pair meets in lanes l and l ^ 16 of a wave
    constexpr int HB = OUT == 2 ? BR / 2 : BR;  // output rows per tile
    const int r0 = tr * HB, c0 = tc * BC;
    const int gbeg = split * p.gps;
    constexpr int KS = CF::KS, SPG = CF::SPG;
    const int nkt = (min(p.G, gbeg + p.gps) - gbeg) * SPG;  // stages of this split
    const int R = p.R, K = p.K, G = p.G;
    const int RW = OUT == 2 ? 2 * R : R;  // weight rows
    // weight row of tile row rt (clamped: rows past the end are never stored)
    auto src_row = [&](int rt) {
        if constexpr (OUT == 2) return ((rt & 16) ? R : 0) + min(r0 + 16 * (rt >> 5) + (rt & 15), R - 1);
        else return min(r0 + rt, R - 1);
    };

    const unsigned lds0 = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)((__attribute__((address_space(3))) unsigned char*)smem));

    // ---- DMA descriptors and per-lane offsets (fixed over K) ----
    const u32x4 rx = make_rsrc(p.X, (unsigned)p.C * K * 2);
    const u32x4 rw = make_rsrc(p.W, (unsigned)RW * (K / 2));
    const unsigned sz_bytes = ((unsigned)RW * G * 2 + 3u) & ~3u;  // see the scale DMA below
    const u32x4 rs = make_rsrc(p.wscale, sz_bytes);
    const u32x4 rz = make_rsrc(p.wzero, sz_bytes);
    int offx[CF::DX], offw[CF::DW];
#pragma unroll
    for (int i = 0; i < CF::DX; ++i) {
        constexpr int CPR = CF::XRB / 16;  // chunks per X row
        const int row = (1024 / CF::XRB) * (wave * CF::DX + i) + lane / CPR;
        offx[i] = (c0 + row) * K * 2 + 16 * ((lane % CPR) ^ swz_x<KS>(row));
    }
#pragma unroll
    for (int i = 0; i < CF::DW; ++i) {
        constexpr int CPR = CF::WRB / 16;  // chunks per weight row
        const int row = (1024 / CF::WRB) * (wave * CF::DW + i) + lane / CPR;
        offw[i] = src_row(row) * (K / 2) + 16 * ((lane % CPR) ^ swz_w<KS>(row));
    }
    // scale / zero: instruction j (of 2 BR / 64) covers rows 64 (j % (BR/64)) + lane,
    // scale for j < BR/64, zero otherwise.  Each lane fetches the aligned dword that
    // holds its fp16; the byte range is rounded up to a dword, a read that stays
    // inside the dword (and so the page) of the array's last element.
    int srow[CF::DS];
#pragma unroll
    for (int i = 0; i < CF::DS; ++i) {
        const int j = wave * CF::DS + i;
        srow[i] = src_row(64 * (j % (BR / 64)) + lane);
    }
    u32x4 rxs = {0u, 0u, 0u, 0u};
    if constexpr (XS) rxs = make_rsrc(p.xs, (unsigned)G * p.ldxs * 4);

    auto issue = [&](int t, int stage) {
        const int u = gbeg * SPG + t;  // stage index along K
        const int g = u / SPG;
        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(stage * SB));
#pragma unroll
        for (int i = 0; i < CF::DX; ++i) dma16(rx, st + (wave * CF::DX + i) * 1024, offx[i], u * CF::XRB);
#pragma unroll
        for (int i = 0; i < CF::DW; ++i)
            dma16(rw, st + OFF_W + (wave * CF::DW + i) * 1024, offw[i], u * CF::WRB);
#pragma unroll
        for (int i = 0; i < CF::DS; ++i) {
            const int j = wave * CF::DS + i;
            const bool is_zero = j >= BR / 64;
            const int voff = ((srow[i] * G + g) * 2) & ~3;
            const unsigned dst = st + (is_zero ? OFF_ZR : OFF_SC) + (j % (BR / 64)) * 256;
            dma4(is_zero ? rz : rs, dst, voff, 0);
        }
        if constexpr (XS) dma4(rxs, st + OFF_XS + wave * 256, (c0 + 64 * wave + lane) * 4, g * p.ldxs * 4);
    };

    // ---- fragment addressing.  Rows of a lane differ between tiles by a
    // multiple of 32, which leaves the swizzle (low row bits) unchanged, so
    // per k-step one per-lane offset serves every tile and the tile enters as
    // an immediate: X row x, step s at 256 x + 16 ((8 h + s) ^ (x & 15));
    // weight row r, half e at 64 r + 16 ((2 h + e) ^ ((r >> 2) & 3)).
    const int h = lane >> 5, l32 = lane & 31;
    const int xrow0 = wc * 32 * FX + l32, wrow0 = wr * 32 * FW + l32;
    unsigned xoff[8];
#pragma unroll
    for (int s = 0; s < KS; ++s) xoff[s] = xrow0 * CF::XRB + 16 * ((KS * h + s) ^ swz_x<KS>(xrow0));
    constexpr int NWC = KS / 4;  // 16-byte weight chunks per lane per stage
    unsigned woff[NWC];
#pragma unroll
    for (int e = 0; e < NWC; ++e) woff[e] = OFF_W + wrow0 * CF::WRB + 16 * ((NWC * h + e) ^ swz_w<KS>(wrow0));
    int wrow[FW];
#pragma unroll
    for (int i = 0; i < FW; ++i) wrow[i] = src_row(wrow0 + 32 * i);

    f32x16 acc[FW][FX];
#pragma unroll
    for (int i = 0; i < FW; ++i)
#pragma unroll
        for (int j = 0; j < FX; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    const f32x16 zero16 = {};

    // ---- prologue: stages 0 .. S-2 in flight ----
#pragma unroll
    for (int t = 0; t < S - 1; ++t)
        if (t < nkt) issue(t, t);

    // stage of tile t (t % S) and of tile t + S - 1 ((t - 1) % S), kept as
    // uniform counters
    int stage = 0, stage_next = S - 1;
    f32x16 P[FW][FX];  // the current group's sums (spans SPG stages)
    for (int t0 = 0; t0 < nkt; t0 += SPG) {
#pragma unroll
    for (int hs = 0; hs < SPG; ++hs) {  // stage hs of the group: compile-time in each copy
        const int t = t0 + hs;
        // stage t landed (everything issued after it may stay in flight), then
        // the barrier: all waves' DMAs of stage t are complete and every wave
        // has finished reading stage t - 1, whose buffer the next issue reuses
        const int ahead = min(S - 2, nkt - 1 - t);
        if (ahead >= 2) wait_vm<vmcnt_imm(2 * D)>();
        else if (ahead == 1) wait_vm<vmcnt_imm(D)>();
        else wait_vm<vmcnt_imm(0)>();
        dma::stage_barrier<0xc07f>();
        if (t + S - 1 < nkt) issue(t + S - 1, stage_next);

        const unsigned st = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(stage * SB));
        stage_next = stage;
        stage = stage + 1 == S ? 0 : stage + 1;
        const int g = gbeg + t / SPG;
        const bool group_first = hs == 0, group_last = hs == SPG - 1;
        // per-lane group scale (x 2^9) and packed -z 2^-9 of the lane's weight rows
        float wsc[FW];
        f16x2 zz[FW];
        const unsigned sbase = st + OFF_SC + wrow0 * 4;
#pragma unroll
        for (int i = 0; i < FW; ++i) {
            const int par = (wrow[i] * G + g) & 1;
            const unsigned sd = lds_read4(sbase + 128 * i);
            const unsigned zd = lds_read4(sbase + (OFF_ZR - OFF_SC) + 128 * i);
            const uint16_t sh = (uint16_t)(par ? (sd >> 16) : (sd & 0xffffu));
            const uint16_t zh = (uint16_t)(par ? (zd >> 16) : (zd & 0xffffu));
            wsc[i] = h2f(sh) * 512.0f;
            const _Float16 nz = (_Float16)(-rintf(h2f(zh)) * (1.0f / 512.0f));
            zz[i] = f16x2{nz, nz};
        }
        u32x4 wraw[FW][NWC];
#pragma unroll
        for (int e = 0; e < NWC; ++e) {
            const unsigned wb = st + woff[e];
#pragma unroll
            for (int i = 0; i < FW; ++i) wraw[i][e] = lds_read16(wb + 32 * CF::WRB * i);
        }

#pragma unroll
        for (int s = 0; s < KS; ++s) {
            f16x8 xf[FX], wf[FW];
            const unsigned xb = st + xoff[s];
#pragma unroll
            for (int j = 0; j < FX; ++j) xf[j] = bitcast<f16x8>(lds_read16(xb + 32 * CF::XRB * j));
#pragma unroll
            for (int i = 0; i < FW; ++i) {
                const u32x4& q = wraw[i][s >> 2];
                const unsigned w = (s & 3) == 0 ? q.x : (s & 3) == 1 ? q.y : (s & 3) == 2 ? q.z : q.w;
                wf[i] = unpack8(w, zz[i]);
            }
#pragma unroll
            for (int i = 0; i < FW; ++i)
#pragma unroll
                for (int j = 0; j < FX; ++j)
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        xf[j], wf[i], (s == 0 && group_first) ? zero16 : P[i][j], 0, 0, 0);
        }

        // ---- fold the group ----
        if (!group_last) continue;
        if constexpr (XS) {
#pragma unroll
            for (int j = 0; j < FX; ++j) {
                float sx[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 v = lds_read16(st + OFF_XS + (wc * 32 * FX + 4 * h) * 4 + (32 * j + 8 * q) * 4);
                    sx[4 * q] = bitcast<float>(v.x);
                    sx[4 * q + 1] = bitcast<float>(v.y);
                    sx[4 * q + 2] = bitcast<float>(v.z);
                    sx[4 * q + 3] = bitcast<float>(v.w);
                }
#pragma unroll
                for (int i = 0; i < FW; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(wsc[i] * sx[v], P[i][j][v], acc[i][j][v]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < FW; ++i)
#pragma unroll
                for (int j = 0; j < FX; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(wsc[i], P[i][j][v], acc[i][j][v]);
        }
    }

    }  // stages of one group
    // ---- split-K: publish, the last arriver sums all partials in split order
    // (not with eight waves: their host plan never splits K) ----
    if constexpr (CF::NW <= 4) {
    if (p.nsplit > 1) {
        constexpr int NC = FW * FX * 4;  // f32x4 chunks per thread
        f32x4 v[NC];
#pragma unroll
        for (int i = 0; i < FW; ++i)
#pragma unroll
            for (int j = 0; j < FX; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[(i * FX + j) * 4 + q] = f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                                    acc[i][j][4 * q + 3]};
        float* slabs = p.part + (size_t)tile * p.nsplit * NC * CF::NT * 4;
        splitk_publish<NC, CF::NT>(slabs + (size_t)split * NC * CF::NT * 4, tid, v);
        // the stages are dead here (every DMA was waited for, every read returned)
        if (!splitk_arrive_is_last(p.counters + tile, (unsigned)p.nsplit, reinterpret_cast<int*>(smem)))
            return;
        splitk_reduce<NC, CF::NT, false>(slabs, p.nsplit, split, tid, v);
#pragma unroll
        for (int i = 0; i < FW; ++i)
#pragma unroll
            for (int j = 0; j < FX; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = v[(i * FX + j) * 4 + q][e];
    }
    }

    // ---- epilogue ----
    if constexpr (OUT == 2) {
        // lane l (l % 32 < 16) holds gate, lane l ^ 16 up, for output row o and
        // the same tokens.  v_permlane16_swap on the accumulators of two tokens
        // (x: token e, y: token e + 1) leaves gate(e) and up(e) in lane l and
        // gate(e + 1) and up(e + 1) in lane l ^ 16: both lanes finish one output.
        const bool up_lane = (l32 & 16) != 0;
#pragma unroll
        for (int i = 0; i < FW; ++i) {
            const int r = r0 + 16 * (wr * FW + i) + (l32 & 15);
#pragma unroll
            for (int j = 0; j < FX; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; e += 2) {
                        const auto sw = __builtin_amdgcn_permlane16_swap(bitcast<unsigned>(acc[i][j][4 * q + e]),
                                                                         bitcast<unsigned>(acc[i][j][4 * q + e + 1]),
                                                                         false, false);
                        const int c = c0 + wc * 32 * FX + 32 * j + 8 * q + 4 * h + e + (up_lane ? 1 : 0);
                        if (r < R && c < p.C)
                            p.out[(int64_t)c * R + r] = swiglu_h(f2h(bitcast<float>(sw[0])), f2h(bitcast<float>(sw[1])));
                    }
        }
        return;
    }
    if constexpr (OUT == 1) {
        // Y[t, o] = alpha acc + beta Y: every old value is loaded first (from a
        // clamped address), then every result stored -- loads and stores to
        // one array in turn would each wait for the previous round trip
        if (p.beta != 0.0f) {
            uint16_t old[FW][FX][16];
#pragma unroll
            for (int i = 0; i < FW; ++i) {
                const int rr = min(r0 + wrow0 + 32 * i, R - 1);
#pragma unroll
                for (int j = 0; j < FX; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int c = c0 + wc * 32 * FX + 32 * j + 8 * (v >> 2) + 4 * h + (v & 3);
                        old[i][j][v] = p.out[(int64_t)min(c, p.C - 1) * R + rr];
                    }
            }
#pragma unroll
            for (int i = 0; i < FW; ++i)
#pragma unroll
                for (int j = 0; j < FX; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        acc[i][j][v] = fmaf(p.beta, h2f(old[i][j][v]), p.alpha * acc[i][j][v]);
        } else {
#pragma unroll
            for (int i = 0; i < FW; ++i)
#pragma unroll
                for (int j = 0; j < FX; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = p.alpha * acc[i][j][v];
        }
    }
#pragma unroll
    for (int i = 0; i < FW; ++i) {
        const int r = r0 + wrow0 + 32 * i;
        if (r >= R) continue;
#pragma unroll
        for (int j = 0; j < FX; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = c0 + wc * 32 * FX + 32 * j + 8 * q + 4 * h;  // 4 consecutive columns
                if constexpr (OUT == 0) {
                    uint16_t* dst = p.out + (int64_t)r * p.C + c;
                    if (c + 3 < p.C && (p.C & 3) == 0) {
                        *reinterpret_cast<u32x2*>(dst) =
                            u32x2{pack2h(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                  pack2h(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c + e < p.C) dst[e] = f2h(acc[i][j][4 * q + e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c + e < p.C) p.out[(int64_t)(c + e) * R + r] = f2h(acc[i][j][4 * q + e]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// B of group-wise INT4 ([K, ldb] bytes, two columns per byte, even n high) ->
// Xt [Npad, K] fp16 = qB - rint(zB[g, n]) (exact), rows n >= N zero, and
// xs [G, Npad] fp32 = sB (0 for n >= N).
//
// A workgroup transposes a 128-k (one group) x 64-byte (128-column) tile
// through LDS: coalesced dword loads of B rows, then thread (column block of
// 8, k block of 8) reads 8 dwords and writes 8 columns x 8 k as 16-byte rows
// of Xt.  K % 128 == 0 (checked by the host).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) i4w_prep_b(const uint8_t* __restrict__ B, int ldb,
                                                  const uint16_t* __restrict__ sB,
                                                  const uint16_t* __restrict__ zB, int N, int K, int G,
                                                  int Npad, uint16_t* __restrict__ Xt,
                                                  float* __restrict__ xs) {
    __shared__ unsigned tile[128][17];  // 128 k-rows x 16 dwords (+1: conflict-free column reads)
    const int tid = threadIdx.x;
    const int g = blockIdx.x, k0 = 128 * g;
    const int b0 = 64 * blockIdx.y;     // first byte column of the tile (column n = 2 b0)
    const bool dw = (ldb & 3) == 0 && (reinterpret_cast<uintptr_t>(B) & 3) == 0;
    // this thread's output columns n0 .. n0 + 7 and k rows 8 k8 .. + 7; their
    // zero points and scales are loaded together with the tile so that the
    // workgroup makes one round trip to memory.  Every load is unconditional,
    // from a clamped address, and masked afterwards: a guarded load becomes a
    // branch whose merge waits for it, which would serialize the round trips.
    const int c8 = tid & 15, k8 = tid >> 4;
    const int n0 = 2 * b0 + 8 * c8;
    uint16_t zh[8], sh16[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int64_t gi = (int64_t)g * N + min(n0 + c, N - 1);
        zh[c] = zB[gi];
        sh16[c] = sB[gi];
    }
    // load: thread t takes row t / 2, dwords 8 (t % 2) .. + 7 of the tile's 64 bytes
    {
        const int r = tid >> 1, d0 = 8 * (tid & 1);
        const uint8_t* row = B + (int64_t)(k0 + r) * ldb;
        unsigned v[8];
        if (dw) {
#pragma unroll
            for (int d = 0; d < 8; ++d)
                v[d] = *reinterpret_cast<const unsigned*>(row + min(b0 + 4 * (d0 + d), ldb - 4));
        } else {
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                unsigned w = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) w |= (unsigned)row[min(b0 + 4 * (d0 + d) + e, ldb - 1)] << (8 * e);
                v[d] = w;
            }
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int bo = b0 + 4 * (d0 + d);
            unsigned w = v[d];
            if (dw) {
                if (bo >= ldb) w = 0;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (bo + e >= ldb) w &= ~(0xffu << (8 * e));
            }
            tile[r][d0 + d] = w;
        }
    }
    __syncthreads();
    // transpose: columns n0 .. n0 + 7 are dword c8 of each row
    if (n0 >= Npad) return;
    unsigned w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = tile[8 * k8 + i][c8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int n = n0 + c;
        const bool in = n < N;
        const float z = in ? rintf(h2f(zh[c])) : 0.0f;
        const int sh = 8 * (c >> 1) + ((c & 1) ? 0 : 4);  // even column: high nibble
        unsigned o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = in ? (float)((w[2 * i] >> sh) & 15u) - z : 0.0f;
            const float b = in ? (float)((w[2 * i + 1] >> sh) & 15u) - z : 0.0f;
            o[i] = pack2h(a, b);
        }
        *reinterpret_cast<u32x4*>(Xt + (int64_t)n * K + k0 + 8 * k8) = u32x4{o[0], o[1], o[2], o[3]};
        if (k8 == 0) xs[(int64_t)g * Npad + n] = in ? h2f(sh16[c]) : 0.0f;
    }
}

}  // namespace i4w
}  // namespace clove
