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
// 1 KB of every group it owns into LDS by LDS DMA at the start and reorders
// it there once, in place: an 8 x 8 nibble transpose (three stages of masked
// swaps of 16-, 8- and 4-bit fields) turns the 8 rows k = 32 q + 8 h .. + 7 of
// 8 columns into one dword per column in the weights' nibble order, stored
// so that lane (h, column) finds the dwords of its four steps in one 16-byte
// slot.  They are unpacked with the same exact (q - z) 2^-9 arithmetic; the
// extra 2^-9 is returned in the fold.
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

// 8 x 8 transpose of 4-bit fields: nibble j of x[i] goes to nibble i of x[j]
// (three stages of field swaps between registers 4, 2 and 1 apart)
__device__ __forceinline__ void nibble_transpose8(unsigned (&x)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned a = x[i], b = x[i + 4];
        x[i] = (a & 0x0000ffffu) | (b << 16);
        x[i + 4] = (a >> 16) | (b & 0xffff0000u);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = (j & 1) + 4 * (j >> 1);  // 0, 1, 4, 5
        const unsigned a = x[i], b = x[i + 2];
        x[i] = (a & 0x00ff00ffu) | ((b << 8) & 0xff00ff00u);
        x[i + 2] = ((a >> 8) & 0x00ff00ffu) | (b & 0xff00ff00u);
    }
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const unsigned a = x[i], b = x[i + 1];
        x[i] = (a & 0x0f0f0f0fu) | ((b << 4) & 0xf0f0f0f0u);
        x[i + 1] = ((a >> 4) & 0x0f0f0f0fu) | (b & 0xf0f0f0f0u);
    }
}

template <class SC, bool XS, int OUT, bool RAWB = false>
__global__ void __launch_bounds__(SC::NT) i4w_stream(Args p) {
    constexpr int WF = SC::WF, XF = SC::XF, NG = SC::NG, D = SC::D, ROWS = SC::ROWS;
    static_assert(!RAWB || (XS && XF == 1), "raw B: group-wise INT4, 16 columns");
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
    // loads group G - 1 and stores none of it.)
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

    // ---- the workgroup's scales, zero points and sx to LDS; their loads go
    // out first, so that waiting for them does not wait for the weight stream
    // issued right behind ----
    constexpr int SPT = 8;  // staged elements per thread per pass
    const int nsz = ROWS * G;
    const int nxs = XS ? G * 16 * XF : 0;
    uint16_t sv[SPT], zv[SPT], sbv[SPT] = {}, zbv[SPT] = {};
    float xv[SPT] = {};
    // unconditional loads from clamped addresses (a guarded load becomes a
    // branch whose merge waits for it, and for everything issued before it)
    auto stage_load = [&](int base) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int idx = base + i * SC::NT + tid;
            const int is = min(idx, nsz - 1);
            const int64_t src = (int64_t)min(r0 + is / G, R - 1) * G + is % G;
            sv[i] = p.wscale[src];
            zv[i] = p.wzero[src];
            if constexpr (RAWB) {
                // sB and zB (converted, and zeroed past N, at the store: a
                // use here would wait for the load before the stream goes out)
                const int e = min(max(idx - nsz, 0), nxs - 1), g = e / 16, c = e % 16;
                const int64_t si = (int64_t)g * p.N + min(c, p.N - 1);
                sbv[i] = p.bscale[si];
                zbv[i] = p.bzero[si];
            } else if constexpr (XS) {
                const int e = min(max(idx - nsz, 0), nxs - 1), g = e / (16 * XF), c = e % (16 * XF);
                xv[i] = p.xs[(int64_t)g * p.ldxs + c];
            }
        }
    };
    auto stage_store = [&](int base) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int idx = base + i * SC::NT + tid;
            if (idx < nsz) {
                lds_s[idx] = sv[i];
                lds_z[idx] = zv[i];
            } else if (XS && idx < nsz + nxs) {
                if constexpr (RAWB) {
                    const bool in = (idx - nsz) % 16 < p.N;
                    lds_xs[idx - nsz] = in ? h2f(sbv[i]) : 0.0f;
                    lds_zb[idx - nsz] = in ? zbv[i] : (uint16_t)0;
                } else {
                    lds_xs[idx - nsz] = xv[i];
                }
            }
        }
    };
    stage_load(0);
    __builtin_amdgcn_sched_barrier(0);  // (keep the order: staging loads, then the stream)
#pragma unroll
    for (int j = 0; j < D; ++j) issue(slot[j], j);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RAWB) {
        // this wave's groups of B to LDS, then from k-row order to step order.
        // In group g, lane l's 16 bytes (rows 2 l, 2 l + 1) go to slot
        // (l + g) % 64.  Unit u = (group, h, half d) reads dword d (columns
        // 8 d .. 8 d + 7, column c at nibble c ^ 1) of the rows
        // k = 32 q + 8 h + r, r < 8, q < 4, of its group and writes column
        // col = 8 d + c's dword of step q to word q of slot 16 h + (col + g) % 16.
        // The rotations by g spread the lanes of every access over the banks:
        // two lanes a bank for the reads, the minimum four passes for the
        // 16-byte writes, and the steps' reads stay one slot a lane.  Only the
        // wave that owns a group touches it here, and one wave's LDS accesses
        // take effect in program order: its copy lands before its reads, and
        // its reads (each write needs all 32 of its lane's reads) before its
        // writes.  The barrier below orders the reorder before the steps.
#pragma unroll
        for (int j = 0; j < NG; ++j)
            if (g0 + j < g1)
                *reinterpret_cast<u32x4*>(lds_b + (g0 + j) * 1024 + ((lane + g0 + j) & 63) * 16) = braw[j];
        for (int u = lane; u < 8 * (g1 - g0); u += 64) {
            const int g = g0 + (u >> 3), hh = (u >> 1) & 3, d = u & 1;
            unsigned char* gb = lds_b + g * 1024;
            unsigned y[4][8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                unsigned x[8];
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    x[r ^ 1] = *reinterpret_cast<const unsigned*>(
                        gb + ((16 * q + 4 * hh + (r >> 1) + g) & 63) * 16 + 8 * (r & 1) + 4 * d);
                nibble_transpose8(x);
#pragma unroll
                for (int c = 0; c < 8; ++c) y[q][c] = x[c ^ 1];
            }
#pragma unroll
            for (int c = 0; c < 8; ++c)
                *reinterpret_cast<u32x4*>(gb + (16 * hh + ((8 * d + c + g) & 15)) * 16) =
                    u32x4{y[0][c], y[1][c], y[2][c], y[3][c]};
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    stage_store(0);
    // (more than SPT elements per thread: rare, and those loads wait behind the stream)
    for (int base = SPT * SC::NT; base < nsz + nxs; base += SPT * SC::NT) {
        stage_load(base);
        stage_store(base);
    }
    __syncthreads();

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
                for (int x = 0; x < XF; ++x)
                    c.sx[x] = *reinterpret_cast<const f32x4*>(lds_xs + g * 16 * XF + 16 * x + 4 * h);
            }
            if constexpr (RAWB) {
                c.zb = lds_zb[g * 16 + l16];
                // column l16, rows k = 128 g + 32 q + 8 h .. + 7 in word q, packed
                // as the weights are (byte j: row 2j high, row 2j + 1 low), in
                // slot 16 h + (l16 + g) % 16
                c.bq = *reinterpret_cast<const u32x4*>(lds_b + g * 1024 + (16 * h + ((l16 + g) & 15)) * 16);
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
                wt[f] = transpose_lane_groups(s.w[f]);
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
                    xq[0] = unpack8(q == 0 ? c.bq.x : q == 1 ? c.bq.y : q == 2 ? c.bq.z : c.bq.w, zzb);
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
                uint16_t* dst = p.out + (int64_t)r * p.C + c;
                if (c + 3 < p.C && (p.C & 3) == 0) {
                    *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(acc[x][f][0], acc[x][f][1]),
                                                           pack2h(acc[x][f][2], acc[x][f][3])};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c + e < p.C) dst[e] = f2h(acc[x][f][e]);
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
