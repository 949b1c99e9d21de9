// Packed INT4 x INT4 GEMM (gemm_int4) for gfx950.
//
// Replaces the reference's gemm_int4 (src/kernels/gemm_int4.cu:45-216).
// Layouts (include/clove/kernels/gemm.cuh:74-87): A_q [M, K/2] with the even k
// in the high nibble; B_q [K, ceil(N/2)] packed along N, even n in the high
// nibble; scales/zeros [M, G] and [G, N], G = ceil(K/128).
//
//  * int4_gemv (N <= 8, the decode shapes) -- one wave streams one weight
//    row with 16-byte loads, the whole row in flight at once.  The per-group
//    integer partials are exact:
//       P = sum qA*qB - zB*sum qA - zA*sum qB + cnt*zA*zB
//    with sum qA*qB from v_dot8_u32_u4 on nibble words, the B words (in A's
//    nibble order) and their chunk sums staged once per workgroup in LDS.
//    Group-wise: acc += (sA*sB) * float(P_g), fp32.
//    Literal: int32 S accumulates sum (qA-8)(qB-8) over all K.
//  * larger N -- the shared MFMA GEMM (mfma_gemm.hpp) with INT4 loaders that
//    unpack both operands to the exact integers q - z in fp16 on their way to
//    LDS; per-group fp32 partials (exact) are scaled by sA*sB after each
//    128-wide group.
#include "common.hpp"
#include "dispatch.hpp"
#include "mfma_gemm.hpp"

#include <type_traits>

namespace clove {
namespace i4 {

using namespace hw;

struct GemvParams {
    const uint8_t* A;
    const uint16_t* A_scale;
    const uint16_t* A_zero;
    const uint8_t* B;
    const uint16_t* B_scale;
    const uint16_t* B_zero;
    uint16_t* C;
    int M, N, K, G;
    int ldb;          // bytes per K row of B
    int cols_valid;   // columns n >= cols_valid read no B (literal: 2*floor(N/2))
    int nch;          // 32-k chunks per row = ceil(K/32)
};

constexpr unsigned kOnes = 0x11111111u;  // eight 4-bit ones

__global__ void fill_u16(uint16_t* p, size_t n, uint16_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// LDS layout (dynamic), per column n < NV:
//   Bw [NV][4*nch] u32   B nibbles of 8 k in A's order (zero for k >= K)
//   Bc [NV][nch]   int4  per 32-k chunk c with cnt valid k, sb = sum qB:
//        group-wise {zB, sb - cnt zB, bits(sB), 0}   literal {64 cnt - 8 sb, 0, 0, 0}
__host__ __device__ inline size_t gemv_lds_bytes(int nv, int nch, int /*G*/) {
    return (size_t)nv * ((size_t)4 * nch * 4 + (size_t)nch * 16);
}

// B nibble word w (k = 8w .. 8w+7) of column n, in A's byte order: byte j holds
// k = 8w + 2j in the high nibble and k = 8w + 2j + 1 in the low nibble
__device__ __forceinline__ unsigned b_word(const GemvParams& p, int n, int w) {
    const int k0 = 8 * w;
    if (n >= p.cols_valid) return 0u;
    if (p.ldb == 1 && k0 + 8 <= p.K && ((reinterpret_cast<uintptr_t>(p.B) + k0) & 7) == 0) {
        // one byte per k row: B[k, 0] in the high nibble, B[k, 1] in the low one
        const u32x2 v = *reinterpret_cast<const u32x2*>(p.B + k0);
        const unsigned ev = __builtin_amdgcn_perm(v.y, v.x, 0x06040200u);  // bytes k0, +2, +4, +6
        const unsigned od = __builtin_amdgcn_perm(v.y, v.x, 0x07050301u);  // bytes k0+1, +3, +5, +7
        if (n == 0) return (ev & 0xf0f0f0f0u) | ((od >> 4) & 0x0f0f0f0fu);
        return ((ev << 4) & 0xf0f0f0f0u) | (od & 0x0f0f0f0fu);
    }
    unsigned word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = k0 + j;
        if (k < p.K) {
            const unsigned byte = p.B[(int64_t)k * p.ldb + (n >> 1)];
            const unsigned nib = (n & 1) ? (byte & 0xfu) : (byte >> 4);
            word |= nib << (8 * (j >> 1) + ((j & 1) ? 0 : 4));
        }
    }
    return word;
}

// Each wave owns RPW consecutive rows of A.  Lane l takes the 16-byte chunks
// c = l + 64u (32 k, a quarter of a 128-k group), u < UPR, of every row; all
// of them (RPW * UPR <= 8 per lane) are loaded before the B staging, so the
// whole weight stream is requested at once.  Per chunk and column the exact integer partial
//     P = sum (qA - zA)(qB - zB) = sum qA qB - zB sum qA - zA (sb - cnt zB)
// is formed with v_dot8_u32_u4 and added to the fp32 accumulator as
// (sA sB) * P.  Literal mode sums (qA - 8)(qB - 8) as int32 over all K.
// Zero points must lie in [-255, 255] (24-bit products).
template <int NV, int MODE, int RPW, int UPR, bool ALIGNED>
__global__ void __launch_bounds__((gemv_max_threads<NV, ALIGNED, 4>())) int4_gemv(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned lds[];
    const int NT = blockDim.x, WPB = NT >> 6;  // UPR: chunks per lane per row per batch
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = p.nch, K = p.K, G = p.G, KW = 4 * nch;
    unsigned* Bw = lds;
    i32x4* Bc = reinterpret_cast<i32x4*>(Bw + NV * KW);  // 16-byte aligned: KW % 4 == 0

    const int row0 = (blockIdx.x * WPB + wave) * RPW;
    int ridx[RPW];  // rows past M read the last row and are not stored
#pragma unroll
    for (int r = 0; r < RPW; ++r) ridx[r] = min(row0 + r, p.M - 1);

    // ---- B for one byte per k row (N <= 2): raw bytes of this thread's 32-k
    // chunks, loaded before the A stream so that waiting for them does not wait
    // for A (loads complete in order) ----
    constexpr int BCH = 2;  // B chunks per thread in the fast path
    const bool bfast = p.ldb == 1 && NV <= 2 && nch <= BCH * NT &&
                       (reinterpret_cast<uintptr_t>(p.B) & 15) == 0 && (K & 31) == 0;
    // (with their groups' B scales and zero points: loaded here, not where the
    // chunk constants are formed, where they would be a second round trip)
    u32x4 braw[BCH][2];
    uint16_t bzr[BCH][NV], bsr[BCH][NV];
    if (bfast) {
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = min(tid + i * NT, nch - 1);  // unconditional, see below
            braw[i][0] = *reinterpret_cast<const u32x4*>(p.B + 32 * c);
            braw[i][1] = *reinterpret_cast<const u32x4*>(p.B + 32 * c + 16);
            if constexpr (MODE == mg::kI4Groupwise) {
#pragma unroll
                for (int n = 0; n < NV; ++n) {
                    const int64_t gi = (int64_t)(c >> 2) * p.N + min(n, p.N - 1);
                    bzr[i][n] = p.B_zero[gi];
                    bsr[i][n] = p.B_scale[gi];
                }
            }
        }
    }

    // A chunks and their group scale / zero.  Loads are unconditional from
    // clamped (valid) addresses and masked where used: a guarded load would
    // become a branch whose merge makes the compiler wait for it right away.
    u32x4 a[RPW][UPR];
    uint16_t sah[RPW][UPR], zah[RPW][UPR];
    auto load_batch = [&](int c0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint8_t* arow = p.A + (int64_t)ridx[r] * (K / 2);
#pragma unroll
            for (int u = 0; u < UPR; ++u) {
                const int cc = min(c0 + 64 * u + lane, nch - 1);
                if constexpr (ALIGNED) {
                    a[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(arow + 16 * cc));
                } else {
                    unsigned w[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        w[d] = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int byte = 16 * cc + 4 * d + e;
                            const unsigned b = (2 * byte < K) ? arow[min(byte, K / 2 - 1)] : 0u;
                            w[d] |= b << (8 * e);
                        }
                    }
                    a[r][u] = u32x4{w[0], w[1], w[2], w[3]};
                }
                if constexpr (MODE == mg::kI4Groupwise) {
                    const int64_t gi = (int64_t)ridx[r] * G + (cc >> 2);
                    sah[r][u] = p.A_scale[gi];
                    zah[r][u] = p.A_zero[gi];
                }
            }
        }
    };
    load_batch(0);

    // ---- stage B once per workgroup ----
    // per-chunk constants of column n (see the LDS layout)
    // (zraw, sraw: column n's B zero point and scale for chunk c's group)
    auto chunk_consts_v = [&](int n, int c, unsigned sb, uint16_t zraw, uint16_t sraw) -> i32x4 {
        const int cnt = min(32, K - 32 * c);
        if constexpr (MODE == mg::kI4Groupwise) {
            const bool in = n < p.N;
            const int zb = in ? (int)rintf(h2f(zraw)) : 0;
            const float sbf = in ? h2f(sraw) : 0.0f;
            return i32x4{zb, (int)sb - cnt * zb, bitcast<int>(sbf), 0};
        } else {
            return i32x4{64 * cnt - 8 * (int)sb, 0, 0, 0};
        }
    };
    auto chunk_consts = [&](int n, int c, unsigned sb) -> i32x4 {
        if constexpr (MODE == mg::kI4Groupwise) {
            const int64_t gi = (int64_t)(c >> 2) * p.N + min(n, p.N - 1);
            return chunk_consts_v(n, c, sb, p.B_zero[gi], p.B_scale[gi]);
        } else {
            return chunk_consts_v(n, c, sb, 0, 0);
        }
    };
    if (bfast) {
        // chunk c: 32 bytes (k = 32c .. 32c+31) -> 4 words per column and its constants
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = tid + i * NT;
            if (c >= nch) continue;
            const unsigned v[8] = {braw[i][0].x, braw[i][0].y, braw[i][0].z, braw[i][0].w,
                                   braw[i][1].x, braw[i][1].y, braw[i][1].z, braw[i][1].w};
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                unsigned w[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const unsigned ev = __builtin_amdgcn_perm(v[2 * d + 1], v[2 * d], 0x06040200u);
                    const unsigned od = __builtin_amdgcn_perm(v[2 * d + 1], v[2 * d], 0x07050301u);
                    w[d] = n == 0 ? ((ev & 0xf0f0f0f0u) | ((od >> 4) & 0x0f0f0f0fu))
                                  : (((ev << 4) & 0xf0f0f0f0u) | (od & 0x0f0f0f0fu));
                    if (n >= p.cols_valid) w[d] = 0u;
                }
                *reinterpret_cast<u32x4*>(Bw + n * KW + 4 * c) = u32x4{w[0], w[1], w[2], w[3]};
                unsigned sb = __builtin_amdgcn_udot8(w[0], kOnes, 0u, false);
                sb = __builtin_amdgcn_udot8(w[1], kOnes, sb, false);
                sb = __builtin_amdgcn_udot8(w[2], kOnes, sb, false);
                sb = __builtin_amdgcn_udot8(w[3], kOnes, sb, false);
                if constexpr (MODE == mg::kI4Groupwise) Bc[n * nch + c] = chunk_consts_v(n, c, sb, bzr[i][n], bsr[i][n]);
                else Bc[n * nch + c] = chunk_consts_v(n, c, sb, 0, 0);
            }
        }
        lds_barrier();
    } else if (NV > 2 && p.ldb <= 4 && (reinterpret_cast<uintptr_t>(p.B) & 15) == 0) {
        // 3 to 8 columns (1 to 4 bytes per k row): word w of every column from
        // rows 8w .. 8w + 7, one vector load for 1, 2 or 4 bytes per row, byte
        // loads for 3 bytes and for the rows of the last word (rows past K
        // read as zero)
        const int ldb = p.ldb;
        for (int w = tid; w < KW; w += NT) {
            const int k0 = 8 * w;
            unsigned rowb[8];  // row j's bytes, byte b of the row at bits 8b
            if (k0 + 8 <= K && ldb != 3) {
                if (ldb == 4) {
                    const u32x4 v0 = *reinterpret_cast<const u32x4*>(p.B + 4 * k0);
                    const u32x4 v1 = *reinterpret_cast<const u32x4*>(p.B + 4 * k0 + 16);
                    rowb[0] = v0.x; rowb[1] = v0.y; rowb[2] = v0.z; rowb[3] = v0.w;
                    rowb[4] = v1.x; rowb[5] = v1.y; rowb[6] = v1.z; rowb[7] = v1.w;
                } else if (ldb == 2) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(p.B + 2 * k0);
                    const unsigned d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) rowb[j] = (d[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                } else {
                    const u32x2 v = *reinterpret_cast<const u32x2*>(p.B + k0);
#pragma unroll
                    for (int j = 0; j < 8; ++j) rowb[j] = ((j < 4 ? v.x : v.y) >> (8 * (j & 3))) & 0xffu;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    unsigned r = 0;
                    if (k0 + j < K)
                        for (int b = 0; b < ldb; ++b) r |= (unsigned)p.B[(int64_t)(k0 + j) * ldb + b] << (8 * b);
                    rowb[j] = r;
                }
            }
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                // column n: byte n / 2 of a row, the high nibble for even n;
                // packed in A's order (byte j: row 2j high, row 2j + 1 low)
                unsigned word = 0;
                if (n < p.cols_valid) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const unsigned nib = (rowb[j] >> (8 * (n >> 1) + ((n & 1) ? 0 : 4))) & 15u;
                        word |= nib << (8 * (j >> 1) + ((j & 1) ? 0 : 4));
                    }
                }
                Bw[n * KW + w] = word;
            }
        }
        lds_barrier();
        for (int idx = tid; idx < NV * nch; idx += NT) {
            const int n = idx / nch, c = idx - n * nch;
            const u32x4 bw = *reinterpret_cast<const u32x4*>(Bw + n * KW + 4 * c);
            unsigned sb = __builtin_amdgcn_udot8(bw.x, kOnes, 0u, false);
            sb = __builtin_amdgcn_udot8(bw.y, kOnes, sb, false);
            sb = __builtin_amdgcn_udot8(bw.z, kOnes, sb, false);
            sb = __builtin_amdgcn_udot8(bw.w, kOnes, sb, false);
            Bc[idx] = chunk_consts(n, c, sb);
        }
        lds_barrier();
    } else {
        for (int idx = tid; idx < NV * KW; idx += NT) Bw[idx] = b_word(p, idx / KW, idx % KW);
        lds_barrier();
        for (int idx = tid; idx < NV * nch; idx += NT) {
            const int n = idx / nch, c = idx - n * nch;
            const u32x4 bw = *reinterpret_cast<const u32x4*>(Bw + n * KW + 4 * c);
            unsigned sb = __builtin_amdgcn_udot8(bw.x, kOnes, 0u, false);
            sb = __builtin_amdgcn_udot8(bw.y, kOnes, sb, false);
            sb = __builtin_amdgcn_udot8(bw.z, kOnes, sb, false);
            sb = __builtin_amdgcn_udot8(bw.w, kOnes, sb, false);
            Bc[idx] = chunk_consts(n, c, sb);
        }
        lds_barrier();
    }

    float accf[RPW][NV];
    int acci[RPW][NV];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int n = 0; n < NV; ++n) { accf[r][n] = 0.0f; acci[r][n] = 0; }

    for (int c0 = 0; c0 < nch; c0 += 64 * UPR) {
        if (c0 > 0) load_batch(c0);
#pragma unroll
        for (int u = 0; u < UPR; ++u) {
            if (c0 + 64 * u >= nch) break;  // uniform across the wave
            const int c = c0 + 64 * u + lane;
            const int cs = min(c, nch - 1);  // lanes past the end compute garbage, masked below
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const bool valid = row0 + r < p.M && c < nch;
                const u32x4 av = a[r][u];
                unsigned sa = __builtin_amdgcn_udot8(av.x, kOnes, 0u, false);
                sa = __builtin_amdgcn_udot8(av.y, kOnes, sa, false);
                sa = __builtin_amdgcn_udot8(av.z, kOnes, sa, false);
                sa = __builtin_amdgcn_udot8(av.w, kOnes, sa, false);
                int za = 0;
                float fa = 0.0f;
                if constexpr (MODE == mg::kI4Groupwise) {
                    za = (int)rintf(h2f(zah[r][u]));
                    fa = valid ? h2f(sah[r][u]) : 0.0f;
                }
#pragma unroll
                for (int n = 0; n < NV; ++n) {
                    const u32x4 bw = *reinterpret_cast<const u32x4*>(Bw + n * KW + 4 * cs);
                    const i32x4 bc = Bc[n * nch + cs];
                    unsigned dot = __builtin_amdgcn_udot8(av.x, bw.x, 0u, false);
                    dot = __builtin_amdgcn_udot8(av.y, bw.y, dot, false);
                    dot = __builtin_amdgcn_udot8(av.z, bw.z, dot, false);
                    dot = __builtin_amdgcn_udot8(av.w, bw.w, dot, false);
                    if constexpr (MODE == mg::kI4Groupwise) {
                        // |terms| < 2^24 for zero points in [-255, 255]: 24-bit products are exact
                        const int P = (int)dot - __mul24(bc.x, (int)sa) - __mul24(za, bc.y);
                        accf[r][n] = fmaf(fa * bitcast<float>(bc.z), (float)P, accf[r][n]);
                    } else {
                        const int P = (int)dot - 8 * (int)sa + bc.x;
                        acci[r][n] += (valid && n < p.cols_valid) ? P : 0;
                    }
                }
            }
        }
    }

    // ---- reduce over the wave (a fixed butterfly, permlane swaps and DPP) ----
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            if constexpr (MODE == mg::kI4Groupwise) accf[r][n] = wave_sum(accf[r][n]);
            else acci[r][n] = wave_sum(acci[r][n]);
        }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = row0 + r;
            if (row >= p.M) break;
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                if (n >= p.N) break;
                float v;
                if constexpr (MODE == mg::kI4Groupwise) {
                    v = accf[r][n];
                } else {
                    const float a_s = h2f(p.A_scale[(int64_t)row * G + (G - 1)]);
                    const float b_s = h2f(p.B_scale[(int64_t)(G - 1) * p.N + n]);
                    v = ((float)acci[r][n] * a_s) * b_s;
                }
                p.C[(int64_t)row * p.N + n] = f2h(v);
            }
        }
    }
}

// One column, group-wise, on rows of 65..128 aligned chunks (K % 32 == 0,
// K = 2080..4096): the KS = ceil(nch / 64) = 2 waves of a workgroup share RPW
// rows of A and split K, wave w taking chunk 64 w + lane of every row.  The lane turns its own 32
// bytes of B (one byte per k, the column in the high nibble) into the four
// nibble words in A's order, their sum and the group's zB / sB in registers --
// nothing is staged in LDS, and that work serves RPW rows -- then forms
// each row's exact chunk partial P as in int4_gemv and (sA sB) * P; each wave
// sums its lanes (the fixed butterfly) and wave 0 adds the KS partials of a
// row in wave order.  Cold graph replays, us per call, against int4_gemv:
// 11008 x 4096 6.83 -> 6.16, 14336 x 4096 8.34 -> 7.15, 11008 x 2304 6.06 ->
// 5.40, 4096 x 4096 4.22 -> 4.18; four rows per workgroup ahead of one, two
// and eight (11008 x 4096: 7.54 / 6.34 / 6.37).  Longer rows (KS 3..8) stay on
// int4_gemv, which measured as fast or faster there (4096 x 11008 6.40 against
// 6.39, 4096 x 14336 7.06 against 7.21, 8192 x 8192 7.80 against 7.71 at best).
// (KS is read from the block size; part[] has room for 8)
template <int RPW>
__global__ void __launch_bounds__(512) int4_gemv_ks(GemvParams p) {
    __shared__ float part[8][RPW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KS = blockDim.x >> 6;
    const int nch = p.nch, K = p.K, G = p.G;
    const int row0 = blockIdx.x * RPW;
    const int c = wave * 64 + lane;
    const int cs = min(c, nch - 1);  // lanes past the end: garbage, masked by sA = 0
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(p.B + 32 * cs);
    const u32x4 b1 = *reinterpret_cast<const u32x4*>(p.B + 32 * cs + 16);
    const uint16_t bz = p.B_zero[cs >> 2], bs = p.B_scale[cs >> 2];
    u32x4 a[RPW];
    uint16_t sah[RPW], zah[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(row0 + r, p.M - 1);
        a[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.A + (int64_t)row * (K / 2) + 16 * cs));
        const int64_t gi = (int64_t)row * G + (cs >> 2);
        sah[r] = p.A_scale[gi];
        zah[r] = p.A_zero[gi];
    }
    // B nibble words in A's order: byte j of word d holds k = 8d + 2j (high) and 8d + 2j + 1 (low)
    const unsigned v[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    unsigned bw[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const unsigned ev = __builtin_amdgcn_perm(v[2 * d + 1], v[2 * d], 0x06040200u);
        const unsigned od = __builtin_amdgcn_perm(v[2 * d + 1], v[2 * d], 0x07050301u);
        bw[d] = (ev & 0xf0f0f0f0u) | ((od >> 4) & 0x0f0f0f0fu);
    }
    unsigned sb = __builtin_amdgcn_udot8(bw[0], kOnes, 0u, false);
    sb = __builtin_amdgcn_udot8(bw[1], kOnes, sb, false);
    sb = __builtin_amdgcn_udot8(bw[2], kOnes, sb, false);
    sb = __builtin_amdgcn_udot8(bw[3], kOnes, sb, false);
    const int zb = (int)rintf(h2f(bz));
    const int sbz = (int)sb - 32 * zb;  // sum (qB - zB) over the chunk
    const float sbf = h2f(bs);
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const bool valid = row0 + r < p.M && c < nch;
        const u32x4 av = a[r];
        unsigned sa = __builtin_amdgcn_udot8(av.x, kOnes, 0u, false);
        sa = __builtin_amdgcn_udot8(av.y, kOnes, sa, false);
        sa = __builtin_amdgcn_udot8(av.z, kOnes, sa, false);
        sa = __builtin_amdgcn_udot8(av.w, kOnes, sa, false);
        unsigned dot = __builtin_amdgcn_udot8(av.x, bw[0], 0u, false);
        dot = __builtin_amdgcn_udot8(av.y, bw[1], dot, false);
        dot = __builtin_amdgcn_udot8(av.z, bw[2], dot, false);
        dot = __builtin_amdgcn_udot8(av.w, bw[3], dot, false);
        const int za = (int)rintf(h2f(zah[r]));
        const float fa = valid ? h2f(sah[r]) : 0.0f;
        // |terms| < 2^24 for zero points in [-255, 255]: 24-bit products are exact
        const int P = (int)dot - __mul24(zb, (int)sa) - __mul24(za, sbz);
        acc[r] = wave_sum((fa * sbf) * (float)P);
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) part[wave][r] = acc[r];
    }
    __syncthreads();
    if (wave != 0 || lane >= RPW) return;
    float t = part[0][lane];
    for (int w = 1; w < KS; ++w) t += part[w][lane];
    const int row = row0 + lane;
    if (row < p.M) p.C[row] = f2h(t);
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kMaxGemvLds = 150 * 1024;

// Rows per wave RPW and waves per workgroup: as many chunk loads per lane in
// flight as fit (8), then workgroups halved until there are two per CU.  Rows
// of 2 x 64 chunks (K 2049..4096) take small workgroups (8 waves of 2 rows):
// the rows then spread over the CUs to within 1.1x of even, where 32-row
// workgroups left some CUs twice the rows of others (11008 x 4096: 6.98 us
// against 7.66, measured).  One or two columns: two workgroups per CU rather
// than one (cold, N = 1: 4096 x 11008 6.67 -> 6.32 us, 4096 x 14336 7.56 ->
// 7.21, 4096 x 4096 4.07 -> 3.88; N = 2: 4096 x 11008 7.46 -> 6.88; seven other
// weight shapes unchanged); with four or eight columns, whose lanes hold more
// registers, one (4096 x 4096 N = 4 6.0 against 6.4 us).
struct GemvShape {
    int rpw, upr, wpb;
};
inline GemvShape gemv_shape(int rows, int nch, int cus, int wg_min) {
    const int cpl = cdiv(nch, 64);
    GemvShape g{1, 8, 16};
    if (cpl >= 7) g = {1, 8, 16};
    else if (cpl >= 5) g = {1, 6, 16};
    else if (cpl >= 3) g = {2, 4, 16};
    else if (cpl == 2) g = {2, 2, 8};
    else g = {8, 1, 16};
    while (g.wpb > 4 && cdiv(rows, g.wpb * g.rpw) < wg_min * cus) g.wpb >>= 1;
    // one chunk per lane per row (K <= 2048): up to two workgroups per CU and
    // one chunk load per row, as for the W4A16 GEMV (w4a16.hip)
    const int target = cpl == 1 ? 2 * cus : cus;
    while (g.rpw > 1 && cdiv(rows, g.wpb * g.rpw) < target) { g.rpw >>= 1; g.upr <<= 1; }
    // a lane never loads more chunks per row than the row has (rounded up to an
    // instantiated width: 1, 2, 4, 6, 8)
    if (g.upr > cpl) g.upr = cpl <= 2 ? cpl : cpl <= 4 ? 4 : cpl <= 6 ? 6 : 8;
    if (g.upr > 8) g.upr = 8;
    return g;
}

template <int NV, int MODE, int RPW, int UPR, bool ALIGNED>
clove_status_t run_gemv_shape(const GemvParams& p, int wpb, hipStream_t stream) {
    const size_t lds = gemv_lds_bytes(NV, p.nch, p.G);
    wpb = min(wpb, gemv_max_threads<NV, ALIGNED, 4>() / 64);
    const dim3 grid(cdiv(p.M, wpb * RPW));
    auto k = int4_gemv<NV, MODE, RPW, UPR, ALIGNED>;
    if (ensure_lds(reinterpret_cast<const void*>(k), (int)lds) != CLOVE_OK) return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, grid, dim3(wpb * 64), lds, stream, p);
    return check_launch();
}

template <int NV, int MODE>
clove_status_t run_gemv(const GemvParams& p, bool aligned, int cus, hipStream_t stream) {
    const GemvShape g = gemv_shape(p.M, p.nch, cus, NV <= 2 ? 2 : 1);
    // unaligned rows are assembled from byte loads (16 registers per chunk
    // until packed): one row per wave and one chunk per lane at a time, so
    // that the variant needs no scratch
    if (!aligned) return run_gemv_shape<NV, MODE, 1, 1, false>(p, g.wpb, stream);
    // (rpw, upr) pairs keep rpw * upr <= 8 chunk loads per lane
    if (g.rpw == 1) {
        if (g.upr >= 8) return run_gemv_shape<NV, MODE, 1, 8, true>(p, g.wpb, stream);
        if (g.upr >= 6) return run_gemv_shape<NV, MODE, 1, 6, true>(p, g.wpb, stream);
        if (g.upr >= 4) return run_gemv_shape<NV, MODE, 1, 4, true>(p, g.wpb, stream);
        if (g.upr >= 2) return run_gemv_shape<NV, MODE, 1, 2, true>(p, g.wpb, stream);
        return run_gemv_shape<NV, MODE, 1, 1, true>(p, g.wpb, stream);
    }
    if (g.rpw == 2) return g.upr >= 4   ? run_gemv_shape<NV, MODE, 2, 4, true>(p, g.wpb, stream)
                           : g.upr >= 2 ? run_gemv_shape<NV, MODE, 2, 2, true>(p, g.wpb, stream)
                                        : run_gemv_shape<NV, MODE, 2, 1, true>(p, g.wpb, stream);
    if (g.rpw == 4) return g.upr >= 2 ? run_gemv_shape<NV, MODE, 4, 2, true>(p, g.wpb, stream)
                                      : run_gemv_shape<NV, MODE, 4, 1, true>(p, g.wpb, stream);
    return run_gemv_shape<NV, MODE, 8, 1, true>(p, g.wpb, stream);
}

// One group-wise column on rows of 65..128 aligned chunks: int4_gemv_ks, four
// rows per workgroup while that leaves two workgroups per CU, else two or one
bool try_gemv_ks(const GemvParams& p, bool aligned, int cus, hipStream_t stream, clove_status_t* st) {
    const int ks = cdiv(p.nch, 64);
    if (p.N != 1 || !aligned || p.ldb != 1 || (reinterpret_cast<uintptr_t>(p.B) & 15) != 0 || ks != 2)
        return false;
    const int rpw = cdiv(p.M, 4) >= 2 * cus ? 4 : cdiv(p.M, 2) >= cus ? 2 : 1;
    const dim3 grid(cdiv(p.M, rpw)), block(64 * ks);
    if (rpw == 4) CLOVE_LAUNCH(int4_gemv_ks<4>, grid, block, 0, stream, p);
    else if (rpw == 2) CLOVE_LAUNCH(int4_gemv_ks<2>, grid, block, 0, stream, p);
    else CLOVE_LAUNCH(int4_gemv_ks<1>, grid, block, 0, stream, p);
    *st = check_launch();
    return true;
}

template <int MODE>
clove_status_t gemv_by_n(const GemvParams& p, bool aligned, int cus, hipStream_t stream) {
    if constexpr (MODE == mg::kI4Groupwise) {
        clove_status_t kst;
        if (try_gemv_ks(p, aligned, cus, stream, &kst)) return kst;
    }
    if (p.N == 1) return run_gemv<1, MODE>(p, aligned, cus, stream);
    if (p.N == 2) return run_gemv<2, MODE>(p, aligned, cus, stream);
    if (p.N <= 4) return run_gemv<4, MODE>(p, aligned, cus, stream);
    return run_gemv<8, MODE>(p, aligned, cus, stream);
}

using mg::Tile;

template <class T, int MODE, bool ALIGNED>
clove_status_t run_mfma(mg::Params p, int cus, hipStream_t stream) {
    using LA = mg::LoadI4Rows<T::BM, T::BK, T::NT, T::LDK, false, MODE, ALIGNED>;
    using LB = mg::LoadI4Cols<T::BN, T::BK, T::NT, T::LDK, MODE, ALIGNED>;
    using EPI = typename std::conditional<MODE == mg::kI4Literal, mg::EpiI4Literal,
                                          mg::EpiAlphaBeta<false>>::type;
    p.tiles_m = cdiv(p.M, T::BM);
    p.tiles_n = cdiv(p.N, T::BN);
    const int tiles = p.tiles_m * p.tiles_n;
    // splits on 128-wide group boundaries so every group is folded whole
    const mg::SplitPlan sp = mg::plan_split(tiles, p.K, 128, cus, 2 * cus, 2);
    p.nsplit = sp.nsplit;
    p.k_per_split = sp.k_per_split;
    if (p.nsplit > 1) {
        Scratch s;
        clove_status_t st = acquire_scratch(stream, (size_t)tiles * p.nsplit * T::BM * T::BN * 4,
                                            (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        p.ws = s.partials;
        p.counters = s.counters;
    }
    constexpr int FOLD = MODE == mg::kI4Literal ? mg::kFoldNone : mg::kFoldAB;
    CLOVE_LAUNCH((mg::mfma_gemm<T, LA, LB, EPI, FOLD>), dim3(tiles * p.nsplit), dim3(T::NT), 0,
                       stream, p);
    return check_launch();
}

template <int MODE>
clove_status_t mfma_by_shape(const mg::Params& p, bool aligned, int cus, hipStream_t stream) {
    if (!aligned) return run_mfma<Tile<64, 64, 64, 2, 2>, MODE, false>(p, cus, stream);
    if (p.N <= 32) return run_mfma<Tile<128, 32, 64, 4, 1>, MODE, true>(p, cus, stream);
    if (p.N <= 64) return run_mfma<Tile<128, 64, 64, 2, 2>, MODE, true>(p, cus, stream);
    return run_mfma<Tile<64, 128, 64, 2, 2>, MODE, true>(p, cus, stream);
}

}  // namespace
}  // namespace i4

clove_status_t launch_gemm_int4(const Int4Args& a, hipStream_t stream) {
    using namespace i4;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const bool literal = a.mode == CLOVE_INT4_REFERENCE_LITERAL;
    const int G = cdiv(a.K, 128);
    const int ldb = literal ? a.N / 2 : (a.N + 1) / 2;
    const int cols_valid = literal ? 2 * (a.N / 2) : a.N;
    const int nch = cdiv(a.K, 32);
    if (a.K == 0) {
        // empty sum: +0 in both modes (the reference reads no scale group then)
        const size_t n = (size_t)a.M * a.N;
        CLOVE_LAUNCH(fill_u16, dim3((unsigned)(n < 1048576 ? cdiv64(n, 256) : 4096)), dim3(256), 0,
                           stream, a.C, n, (uint16_t)0);
        return check_launch();
    }
    if (a.N <= 8 && gemv_lds_bytes(a.N <= 2 ? a.N : (a.N <= 4 ? 4 : 8), nch, G) <= kMaxGemvLds) {
        GemvParams p{a.A, a.A_scale, a.A_zero, a.B, a.B_scale, a.B_zero, a.C,
                     a.M, a.N, a.K, G, ldb, cols_valid, nch};
        const bool aligned = aligned16(a.A) && (a.K % 32 == 0);
        return literal ? gemv_by_n<mg::kI4Literal>(p, aligned, dev.num_cus, stream)
                       : gemv_by_n<mg::kI4Groupwise>(p, aligned, dev.num_cus, stream);
    }
    if (!literal) {
        clove_status_t st2;
        if (try_i4i4(a, dev.num_cus, stream, &st2)) return st2;
        if (try_i4w_int4(a, dev.num_cus, stream, &st2)) return st2;
    }
    mg::Params p{};
    p.a = a.A; p.a_scale = a.A_scale; p.a_zero = a.A_zero;
    p.b = a.B; p.b_scale = a.B_scale; p.b_zero = a.B_zero;
    p.c = a.C;
    p.M = a.M; p.N = a.N; p.K = a.K; p.G = G;
    p.ldb_bytes = ldb;
    p.b_cols_valid = cols_valid;
    p.alpha = 1.0f; p.beta = 0.0f;
    const bool aligned = aligned16(a.A) && (a.K % 32 == 0) && (reinterpret_cast<uintptr_t>(a.B) % 8 == 0) &&
                         (ldb % 8 == 0);
    return literal ? mfma_by_shape<mg::kI4Literal>(p, aligned, dev.num_cus, stream)
                   : mfma_by_shape<mg::kI4Groupwise>(p, aligned, dev.num_cus, stream);
}

}  // namespace clove
