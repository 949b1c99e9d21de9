// Streaming MFMA GEMM with packed INT4 weight rows for few X rows (C <= 32):
// group-wise INT4 with N in 9..32 columns and W4A16 with 5..32 tokens.  The
// same arithmetic as i4w_gemm (i4w_gemm.hpp):
//
//   out[r, c] = sum_g  sw[r,g] * sx[g,c] * P_g[r,c]
//   P_g[r,c]  = sum_{k in group g} (q[r,k] - zw[r,g]) * x[c,k]        (exact)
//
// shaped for the weight stream: no LDS stages and no barriers in the K loop.
// A workgroup of KS waves owns 16 WF weight rows; wave w takes groups
// [w gq, (w+1) gq) of K and loads its rows' 64-byte group slices straight into
// VGPRs, D groups ahead of the one it computes, so that the whole weight
// matrix is in flight across the grid at once.  X (shared by every workgroup,
// served by L2) is loaded the same way.  The workgroup's scales, zero points
// (and sx) are copied to LDS once at the start; the KS partial sums of an
// output meet in LDS once at the end, in wave order.
//
// One v_mfma_f32_16x16x32_f16 per (16 X rows, 16 weight rows, 32 k): the X
// fragment is the "A" operand (lane l: X row l % 16) and the weight fragment
// the "B" operand (lane l: weight row l % 16), so each lane owns one weight
// row and four X rows of the result.  In step q of a group, lane group
// h = l / 16 holds k = 32 q + 8 h .. + 7, so that the four lane groups of one
// X load read 64 contiguous bytes of a row.  A weight row's group slice
// arrives as one 16-byte load per lane (lane group h: k = 32 h .. 32 h + 31,
// dword j = k 32 h + 8 j) and a 4 x 4 transpose across lane groups and
// dwords (v_permlane16_swap, then v_permlane32_swap) gives lane group h the
// dwords of k = 32 q + 8 h.
//
// RAWB (group-wise INT4 with 15 or 16 columns): no transpose pre-pass.  B
// [K, 8] bytes (16 nibbles per k row) is contiguous, so each wave copies the
// 1 KB of every group it owns into LDS in k-row order at the start, and
// gfx950's ds_read_b64_tr_b4 transposes it on the way out: within a 16-lane
// group, result lane j gets nibble j of the 16 source lanes' 8-byte rows,
// i.e. 16 consecutive k of one column (nibble j of a row is column j ^ 1: the
// even column sits in the high nibble), so lane l's X row is column
// (l % 16) ^ 1.  Two such reads give lane group h the k = 32 h .. 32 h + 31 of
// the group, and step q uses k = 32 h + 8 q .. + 7 -- the order in which the
// weights' 16-byte group slices arrive, so with raw B the weights need no
// lane-group transpose either.  B nibbles come out with the even k in the
// low nibble (unpack8<true>), and are unpacked with the same exact
// (q - z) 2^-9 arithmetic; the extra 2^-9 is returned in the fold.
#pragma once

#include "i4w_gemm.hpp"

namespace clove {
namespace i4w {

// WF: 16-row weight fragments per wave, XF: 16-row X fragments (C <= 16 XF),
// NG: groups per wave (gq <= NG), KS: waves (K slices) per workgroup,
// D: groups in flight ahead of the computed one
template <int WF_, int XF_, int NG_, int KS_, int D_ = 4>
struct SCfg {
    static constexpr int WF = WF_, XF = XF_, NG = NG_, KS = KS_, D = D_ < NG_ ? D_ : NG_;
    static constexpr int NT = 64 * KS, ROWS = 16 * WF;
    // partial sums of the KS waves, then the workgroup's scales and zero
    // points ([ROWS][G] fp16 each) and sx ([G][16 XF] fp32)
    static constexpr int RED_BYTES = KS * XF * WF * 4 * 64 * 4;
    static constexpr int lds_bytes(int G, bool xs, bool rawb = false) {
        return RED_BYTES + 2 * ((ROWS * G * 2 + 15) & ~15) + (xs ? G * 16 * XF * 4 : 0) +
               (rawb ? ((G * 16 * 2 + 15) & ~15) + G * 1024 : 0);
    }
};

// lane group h of (r0, r1, r2, r3) holds dwords 4 h .. 4 h + 3 of a 16-dword
// block; afterwards register q holds dword 4 q + h
__device__ __forceinline__ u32x4 transpose_lane_groups(u32x4 v) {
    const auto a = __builtin_amdgcn_permlane16_swap(v.x, v.y, false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(v.z, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
    return u32x4{c[0], d[0], c[1], d[1]};
}

typedef int i32x2v __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) i32x2v lds_i32x2v;

// ds_read_b64_tr_b4 at LDS byte address a (see the RAWB note above)
__device__ __forceinline__ u32x2 lds_read_tr4(unsigned a) {
    const i32x2v v = __builtin_amdgcn_ds_read_tr4_b64_v2i32(reinterpret_cast<lds_i32x2v*>((size_t)a));
    return u32x2{(unsigned)v[0], (unsigned)v[1]};
}

template <class SC, bool XS, int OUT, bool RAWB = false>
__global__ void __launch_bounds__(SC::NT) i4w_stream(Args p) {
    constexpr int WF = SC::WF, XF = SC::XF, NG = SC::NG, D = SC::D, ROWS = SC::ROWS;
    static_assert(!RAWB || (XS && XF == 1 && OUT == 0), "raw B: group-wise INT4, 16 columns");
    extern __shared__ __attribute__((aligned(16))) float red[];

    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 4, l16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int R = p.R, K = p.K, G = p.G;
    const int r0 = blockIdx.x * ROWS;
    const int gq = (G + SC::KS - 1) / SC::KS;
    const int g0 = wave * gq, g1 = min(G, g0 + gq);  // this wave's groups (none when g0 >= G)
    uint16_t* lds_s = reinterpret_cast<uint16_t*>(reinterpret_cast<unsigned char*>(red) + SC::RED_BYTES);
    uint16_t* lds_z = lds_s + ((ROWS * G + 7) & ~7);
    float* lds_xs = reinterpret_cast<float*>(lds_z + ((ROWS * G + 7) & ~7));
    uint16_t* lds_zb = reinterpret_cast<uint16_t*>(lds_xs + (XS ? G * 16 * XF : 0));  // RAWB: zB [G][16]
    unsigned char* lds_b = reinterpret_cast<unsigned char*>(lds_zb) + ((G * 16 * 2 + 15) & ~15);  // RAWB: B

    const uint8_t* wrow[WF];
#pragma unroll
    for (int f = 0; f < WF; ++f)  // rows past R read the last row and are never stored
        wrow[f] = p.W + (int64_t)min(r0 + 16 * f + l16, R - 1) * (K / 2) + 16 * h;
    const uint16_t* xrow[XF];
#pragma unroll
    for (int j = 0; j < XF; ++j)
        xrow[j] = RAWB ? nullptr : p.X + (int64_t)min(16 * j + l16, p.C - 1) * K + 8 * h;

    // RAWB: this wave's groups of B (1 KB each: 128 k rows x 8 bytes), 16
    // bytes a lane, loaded ahead of every other load.  Ordinary loads, not LDS
    // DMA: loads complete in order, so the wait for these waits for nothing
    // issued after them, where a read of LDS behind an LDS DMA waits for every
    // outstanding load, the weight stream included.  (A wave without groups
    // loads group G - 1, see the staging below.)
    u32x4 braw[RAWB ? NG : 1];
    if constexpr (RAWB) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int g = max(0, min(g0 + j, g1 - 1));
            braw[j] = *reinterpret_cast<const u32x4*>(p.B + (int64_t)g * 1024 + 16 * lane);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    struct Slot {
        u32x4 w[WF];
        f16x8 x[XF][4];
    };
    Slot slot[D];
    auto issue = [&](Slot& s, int j) {
        const int g = max(0, min(g0 + j, g1 - 1));
#pragma unroll
        for (int f = 0; f < WF; ++f)
            s.w[f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[f] + 64 * g));
        if constexpr (!RAWB) {
#pragma unroll
            for (int x = 0; x < XF; ++x)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    s.x[x][q] = *reinterpret_cast<const f16x8*>(xrow[x] + 128 * g + 32 * q);
        }
    };

    // ---- this wave's scales and zero points (and sx, or sB / zB) to LDS.
    // Every wave stages exactly the constants of the groups it computes (a
    // wave without groups those of group G - 1, the same values its owner
    // writes), so no wave waits for another before its K loop: one wave's LDS
    // accesses take effect in program order.  The loads go out first, so that
    // waiting for them does not wait for the weight stream issued right
    // behind; they are unconditional, from clamped addresses (a guarded load
    // becomes a branch whose merge waits for it, and for everything issued
    // before it) ----
    const int gs0 = g0 < G ? g0 : G - 1;      // first staged group
    const int ngs = g0 < G ? g1 - g0 : 1;     // staged groups, 1..NG
    constexpr int SPL = (ROWS * NG + 63) / 64;                 // weight constants per lane
    constexpr int XPL = XS ? (16 * XF * NG + 63) / 64 : 1;     // sx entries per lane
    uint16_t sv[SPL], zv[SPL], sbv[XPL] = {}, zbv[XPL] = {};
    float xv[XPL] = {};
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const int e = min(lane + 64 * i, ROWS * NG - 1), row = e / NG, gj = min(e % NG, ngs - 1);
        const int64_t src = (int64_t)min(r0 + row, R - 1) * G + gs0 + gj;
        sv[i] = p.wscale[src];
        zv[i] = p.wzero[src];
    }
    if constexpr (XS) {
#pragma unroll
        for (int i = 0; i < XPL; ++i) {
            const int e = min(lane + 64 * i, 16 * XF * NG - 1), gj = min(e / (16 * XF), ngs - 1), c = e % (16 * XF);
            if constexpr (RAWB) {
                // sB and zB (converted, and zeroed past N, at the store: a use
                // here would wait for the load before the stream goes out)
                const int64_t si = (int64_t)(gs0 + gj) * p.N + min(c, p.N - 1);
                sbv[i] = p.bscale[si];
                zbv[i] = p.bzero[si];
            } else {
                xv[i] = p.xs[(int64_t)(gs0 + gj) * p.ldxs + c];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // (keep the order: staging loads, then the stream)
#pragma unroll
    for (int j = 0; j < D; ++j) issue(slot[j], j);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RAWB) {
        // this wave's groups of B to LDS in k-row order, 8 bytes a row, with
        // the two 16-row halves of every odd 32-row block swapped (lane l's 16
        // bytes are rows 2 l and 2 l + 1; chunk l goes to chunk l ^ 8 when bit
        // 4 of l is set): a transposing read of lane group h covers 16 rows of
        // block h, and with the swap the four lane groups of one read fall on
        // alternate 128-byte halves of the banks (two passes, the minimum for
        // 512 bytes)
#pragma unroll
        for (int j = 0; j < NG; ++j)
            if (j < ngs)
                *reinterpret_cast<u32x4*>(lds_b + (gs0 + j) * 1024 + (lane ^ (((lane >> 4) & 1) << 3)) * 16) = braw[j];
    }
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const int e = lane + 64 * i, row = e / NG, gj = e % NG;
        if (e < ROWS * NG && gj < ngs) {
            lds_s[row * G + gs0 + gj] = sv[i];
            lds_z[row * G + gs0 + gj] = zv[i];
        }
    }
    if constexpr (XS) {
#pragma unroll
        for (int i = 0; i < XPL; ++i) {
            const int e = lane + 64 * i, gj = e / (16 * XF), c = e % (16 * XF);
            if (e < 16 * XF * NG && gj < ngs) {
                const int d = (gs0 + gj) * 16 * XF + c;
                if constexpr (RAWB) {
                    const bool in = c < p.N;
                    lds_xs[d] = in ? h2f(sbv[i]) : 0.0f;
                    lds_zb[d] = in ? zbv[i] : (uint16_t)0;
                } else {
                    lds_xs[d] = xv[i];
                }
            }
        }
    }
    const unsigned lds_b_addr = (unsigned)(size_t)((__attribute__((address_space(3))) unsigned char*)lds_b);
    // (the K loop's LDS reads stay behind these stores)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    f32x4 acc[XF][WF];
#pragma unroll
    for (int j = 0; j < XF; ++j)
#pragma unroll
        for (int f = 0; f < WF; ++f) acc[j][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    {
        // groups past g1 reload the last one (an L2 hit; a wave without groups
        // reloads group G - 1) and fold with scale 0: straight-line code, so
        // every wait the compiler places is for one slot.
        //
        // The group's LDS constants (weight zero points and scales, sx, and
        // for raw B its zero points and the lane's 16-byte slot), read one
        // group ahead: a group's unpack and MFMAs then never wait for an LDS
        // round trip
        struct Cst {
            uint16_t z[WF], s[WF];
            f32x4 sx[XS ? XF : 1];
            uint16_t zb;
            u32x4 bq;
        };
        auto load_cst = [&](int j) {
            Cst c{};
            const int g = max(0, min(g0 + j, g1 - 1));
#pragma unroll
            for (int f = 0; f < WF; ++f) {
                c.z[f] = lds_z[(16 * f + l16) * G + g];
                c.s[f] = lds_s[(16 * f + l16) * G + g];
            }
            if constexpr (XS) {
#pragma unroll
                for (int x = 0; x < XF; ++x) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(lds_xs + g * 16 * XF + 16 * x + 4 * h);
                    // raw B: accumulator row 4 h + e is column 4 h + (e ^ 1)
                    c.sx[x] = RAWB ? f32x4{v[1], v[0], v[3], v[2]} : v;
                }
            }
            if constexpr (RAWB) {
                c.zb = lds_zb[g * 16 + (l16 ^ 1)];
                // column l16 ^ 1, rows k = 128 g + 32 h + 8 q .. + 7 in word q
                // (two transposing reads of 16 rows; odd blocks h have their
                // halves swapped, see the copy above)
                const unsigned gb = lds_b_addr + g * 1024;
                const int sw = (h & 1) << 4;
                const u32x2 lo = lds_read_tr4(gb + 8 * ((32 * h + l16) ^ sw));
                const u32x2 hi = lds_read_tr4(gb + 8 * ((32 * h + 16 + l16) ^ sw));
                c.bq = u32x4{lo.x, lo.y, hi.x, hi.y};
            }
            return c;
        };
        auto compute = [&](const Slot& s, const Cst& c, int j) {
            const bool valid = g0 + j < g1;
            f32x4 P[XF][WF];
            u32x4 wt[WF];
            f16x2 zz[WF];
#pragma unroll
            for (int f = 0; f < WF; ++f) {
                // (raw B takes the k order in which the slices arrive)
                wt[f] = RAWB ? s.w[f] : transpose_lane_groups(s.w[f]);
                const _Float16 nz = (_Float16)(-rintf(h2f(c.z[f])) * (1.0f / 512.0f));
                zz[f] = f16x2{nz, nz};
            }
            f16x2 zzb;
            if constexpr (RAWB) {
                const _Float16 nzb = (_Float16)(-rintf(h2f(c.zb)) * (1.0f / 512.0f));
                zzb = f16x2{nzb, nzb};
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                f16x8 xq[XF];
                if constexpr (RAWB) {
                    xq[0] = unpack8<true>(q == 0 ? c.bq.x : q == 1 ? c.bq.y : q == 2 ? c.bq.z : c.bq.w, zzb);
                } else {
#pragma unroll
                    for (int x = 0; x < XF; ++x) xq[x] = s.x[x][q];
                }
#pragma unroll
                for (int f = 0; f < WF; ++f) {
                    const unsigned wd = q == 0 ? wt[f].x : q == 1 ? wt[f].y : q == 2 ? wt[f].z : wt[f].w;
                    const f16x8 wf = unpack8(wd, zz[f]);
#pragma unroll
                    for (int x = 0; x < XF; ++x)
                        P[x][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            xq[x], wf, q == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : P[x][f], 0, 0, 0);
                }
            }
#pragma unroll
            for (int f = 0; f < WF; ++f) {
                // (q - z) 2^-9 back to q - z; 0 for the reloaded tail groups
                const float wsc = valid ? h2f(c.s[f]) * (RAWB ? 262144.0f : 512.0f) : 0.0f;
#pragma unroll
                for (int x = 0; x < XF; ++x) {
                    f32x4 sc = {wsc, wsc, wsc, wsc};
                    if constexpr (XS) sc = sc * c.sx[x];
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[x][f][e] = fmaf(sc[e], P[x][f][e], acc[x][f][e]);
                }
            }
        };
        // sched_barrier: keep the loads where they are written (the scheduler
        // would sink them toward their use to save registers, which shortens
        // the prefetch to nothing)
        Cst cur = load_cst(0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            // (past the last group: a harmless reread of the last group's constants)
            const Cst nxt = load_cst(j + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(slot[j % D], cur, j);
            __builtin_amdgcn_sched_barrier(0);
            if (j + D < NG) issue(slot[j % D], j + D);
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
        }
    }

    // ---- the KS partials of each output, summed in wave order ----
    constexpr int NV = XF * WF * 4;
    if constexpr (SC::KS > 1) {
#pragma unroll
        for (int x = 0; x < XF; ++x)
#pragma unroll
            for (int f = 0; f < WF; ++f)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[((wave * NV) + (x * WF + f) * 4 + e) * 64 + lane] = acc[x][f][e];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int x = 0; x < XF; ++x)
#pragma unroll
            for (int f = 0; f < WF; ++f)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = acc[x][f][e];
                    for (int w = 1; w < SC::KS; ++w) v += red[((w * NV) + (x * WF + f) * 4 + e) * 64 + lane];
                    acc[x][f][e] = v;
                }
    }

    // ---- epilogue: lane holds weight row r0 + 16 f + l16 and X rows 16 x + 4 h .. + 3 ----
    if constexpr (OUT == 1) {
        // every old value of Y first (clamped addresses), then every store: a
        // load after a store to the same array would wait for a round trip each
        if (p.beta != 0.0f) {
            uint16_t old[XF][WF][4];
#pragma unroll
            for (int f = 0; f < WF; ++f)
#pragma unroll
                for (int x = 0; x < XF; ++x)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        old[x][f][e] = p.out[(int64_t)min(16 * x + 4 * h + e, p.C - 1) * R +
                                             min(r0 + 16 * f + l16, R - 1)];
#pragma unroll
            for (int f = 0; f < WF; ++f)
#pragma unroll
                for (int x = 0; x < XF; ++x)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[x][f][e] = fmaf(p.beta, h2f(old[x][f][e]), p.alpha * acc[x][f][e]);
        } else {
#pragma unroll
            for (int f = 0; f < WF; ++f)
#pragma unroll
                for (int x = 0; x < XF; ++x)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[x][f][e] = p.alpha * acc[x][f][e];
        }
    }
#pragma unroll
    for (int f = 0; f < WF; ++f) {
        const int r = r0 + 16 * f + l16;
        if (r >= R) continue;
#pragma unroll
        for (int x = 0; x < XF; ++x) {
            const int c = 16 * x + 4 * h;
            if constexpr (OUT == 0) {
                // (raw B: accumulator entry e is column c + (e ^ 1))
                constexpr int SW = RAWB ? 1 : 0;
                uint16_t* dst = p.out + (int64_t)r * p.C + c;
                if (c + 3 < p.C && (p.C & 3) == 0) {
                    *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(acc[x][f][0 ^ SW], acc[x][f][1 ^ SW]),
                                                           pack2h(acc[x][f][2 ^ SW], acc[x][f][3 ^ SW])};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c + e < p.C) dst[e] = f2h(acc[x][f][e ^ SW]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < p.C) p.out[(int64_t)(c + e) * R + r] = f2h(acc[x][f][e]);
            }
        }
    }
}

}  // namespace i4w
}  // namespace clove
