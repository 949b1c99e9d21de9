// W4A16 linear layer for gfx950: Y = alpha * X @ dequant(W)^T + beta * Y.
//
// X [T,K] fp16 activations, W_q [O, K/2] group-128 INT4 weights in gemm_int4's
// A layout (src/kernels/gemm_int4.cu:27-34: even k in the high nibble), scales
// and zeros [O, G].  It is the reference runtime's linear-layer call
// (src/runtime/inference.cu:139-194, beta = 1 residual at :165-168, :191-194)
// on INT4 weights.
//
//  * w4a16_gemv (T <= 2, and T = 3, 4 on small weights: decode) -- a wave
//    streams one or more weight rows with 16-byte loads, all in flight at once; the nibbles are turned into the
//    exact fp16 integers q - z and dotted with X (staged in LDS, or for one
//    token on rows of up to 2048 k loaded per lane into registers, where the
//    zero point comes off once per chunk) by v_dot2_f32_f16 in fp32;
//    acc += scale * that per 32-k chunk.
//  * larger T -- the INT4-weight MFMA GEMM (i4w_gemm.hpp) when K % 128 == 0
//    and the operands are aligned, else the shared MFMA GEMM (mfma_gemm.hpp):
//    X rows as operand A, W rows unpacked to the exact integers q - z as
//    operand B; the per-group fp32 partials are scaled by s[o,g] after each
//    128-wide group.
//
// launch_w4a16_swiglu: the MLP's gate and up projections and SwiGLU in one
// pass over a fused [2 O, K/2] weight (gate rows, then up rows): the GEMV and
// the MFMA GEMM pair each gate row with its up row inside a workgroup, so
// neither projection is written to memory.
#include "common.hpp"
#include "dispatch.hpp"
#include "mfma_gemm.hpp"

namespace clove {
namespace w4 {

using namespace hw;

struct GemvParams {
    const uint16_t* X;
    const uint8_t* W;
    const uint16_t* scale;
    const uint16_t* zero;
    uint16_t* Y;
    int T, O, K, G;
    int nch;  // ceil(K/32)
    float alpha, beta;
};

// LDS (dynamic): Xs [TV][32*nch] fp16, zero past K, each 8-k block stored in
// the order x0 x2 x4 x6 x1 x3 x5 x7 (the order the weight pairs come out of
// the nibble unpack below)
__host__ __device__ inline size_t gemv_lds_bytes(int tv, int nch) { return (size_t)tv * 32 * nch * 2; }

// X position of k inside its 8-k block: even k first, then odd k
__host__ __device__ constexpr int xperm(int k) { return (k & ~7) | ((k & 1) << 2) | ((k & 7) >> 1); }

// Each wave owns RPW consecutive weight rows; lane l takes the 16-byte chunks
// c = l + 64u (32 k), u < UPR, of every row, all loaded up front (X is staged
// first so that waiting for it does not wait for the weights).  A weight dword
// holds k = 8d..8d+7 with the even k in the high nibbles: the nibbles become
// the fp16 values 1024 + q (v_perm against 0x64 bytes), minus 1024 + z gives
// q - z exactly, and v_dot2_f32_f16 with the X pairs accumulates
// sum_k x_k (q_k - z) in fp32 with exact products; acc += s * that per chunk.
//
// DX (one token, one aligned chunk per lane, K % 32 == 0, 16-byte aligned X):
// no LDS.  Each lane loads the 32 x of its own chunk straight into registers
// (they serve every row of the wave), permutes them into the unpack order
// there and sums them once (sx, fp32); the rows then dot x with 1024 + q and
// subtract (1024 + z) * sx per chunk, which takes the per-weight zero-point
// subtraction out of the inner loop.  The products are still exact; the fp32
// sums carry the 1024 offset (relative to the chunk's sum of |x| the rounding
// is ~2^-24 * 1039).  Integer-valued x and q - z stay exact below 2^24.
//
// SWIGLU: the weight holds 2 O rows (gate rows 0..O-1, then up rows O..2O-1)
// and the output is H [T, O] = swiglu(fp16(gate), fp16(up)); a wave takes RPW/2
// gate rows and the RPW/2 up rows of the same outputs, so the pair meets in
// one lane's registers.
// Threads per workgroup: as for the other GEMVs, except that four rows of two
// chunks each (and their scales / zero points) need more than the 128 VGPRs a
// 1024-thread workgroup leaves
template <int TV, int RPW, int UPR, bool ALIGNED>
__host__ __device__ constexpr int w4_max_threads() {
    return (RPW >= 4 && UPR >= 2) ? 512 : gemv_max_threads<TV, ALIGNED, 2>();
}

template <int TV, int RPW, int UPR, bool ALIGNED, bool SWIGLU = false, bool DX = false>
__global__ void __launch_bounds__((w4_max_threads<TV, RPW, UPR, ALIGNED>())) w4a16_gemv(GemvParams p) {
    static_assert(!SWIGLU || RPW % 2 == 0, "gate / up row pairs");
    static_assert(!DX || (TV == 1 && UPR == 1 && ALIGNED && RPW <= 4), "direct X: one token, one chunk per lane");
    constexpr int LR = SWIGLU ? RPW / 2 : RPW;  // output rows per wave
    extern __shared__ __attribute__((aligned(16))) unsigned lds[];
    const int NT = blockDim.x, WPB = NT >> 6;  // waves per workgroup (rows / RPW)
    constexpr int XPT = 4;  // X prefetch: 16-byte pieces per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = p.nch, K = p.K, G = p.G, KP = 32 * nch;
    uint16_t* Xs = reinterpret_cast<uint16_t*>(lds);

    const int row0 = (blockIdx.x * WPB + wave) * LR;  // first output row of the wave
    int ridx[RPW];  // weight rows; rows past O read the last row and are not stored
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        ridx[r] = (SWIGLU && r >= LR) ? p.O + min(row0 + r - LR, p.O - 1) : min(row0 + r % LR, p.O - 1);

    // ---- X: 16-byte pieces (8 k) into registers first (the first XPT per
    // thread; with several tokens, any further pieces are loaded at the
    // staging -- one token always fits for K <= 32768) ----
    const int npieces = TV * KP / 8;
    const bool xfast = !DX && (TV > 1 || npieces <= XPT * NT) && (K & 7) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.X) & 15) == 0;
    u32x4 xr[XPT];
    if constexpr (DX) {
        // the lane's chunk (nch <= 64: lanes past the end reload the last one)
        const int cs = min(lane, nch - 1);
#pragma unroll
        for (int d = 0; d < 4; ++d) xr[d] = *reinterpret_cast<const u32x4*>(p.X + 32 * cs + 8 * d);
    } else if (xfast) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
            const int q = min(tid + i * NT, npieces - 1);
            const int t = q / (KP / 8), k8 = (q - t * (KP / 8)) * 8;
            const int tt = min(t, p.T - 1), kk = min(k8, K - 8);
            xr[i] = *reinterpret_cast<const u32x4*>(p.X + (int64_t)tt * K + kk);
        }
    }

    // ---- the weight chunks and their group scale / zero (unconditional
    // clamped loads, masked where used) ----
    u32x4 a[RPW][UPR];
    uint16_t sh[RPW][UPR], zh[RPW][UPR];
    auto load_batch = [&](int c0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint8_t* wrow = p.W + (int64_t)ridx[r] * (K / 2);
#pragma unroll
            for (int u = 0; u < UPR; ++u) {
                const int cc = min(c0 + 64 * u + lane, nch - 1);
                if constexpr (ALIGNED) {
                    a[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + 16 * cc));
                } else {
                    unsigned w[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        w[d] = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int byte = 16 * cc + 4 * d + e;
                            const unsigned b = (2 * byte < K) ? wrow[min(byte, K / 2 - 1)] : 0u;
                            w[d] |= b << (8 * e);
                        }
                    }
                    a[r][u] = u32x4{w[0], w[1], w[2], w[3]};
                }
                const int64_t gi = (int64_t)ridx[r] * G + (cc >> 2);
                sh[r][u] = p.scale[gi];
                zh[r][u] = p.zero[gi];
            }
        }
    };
    load_batch(0);

    // ---- stage X in the permuted order ----
    if constexpr (DX) {
    } else if (xfast) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
            const int q = tid + i * NT;
            if (q >= npieces) continue;
            const int t = q / (KP / 8), k8 = (q - t * (KP / 8)) * 8;
            u32x4 v = xr[i];
            if (t >= p.T || k8 >= K) v = u32x4{0u, 0u, 0u, 0u};
            // (x0 x1)(x2 x3)(x4 x5)(x6 x7) -> (x0 x2)(x4 x6)(x1 x3)(x5 x7)
            const u32x4 o = {__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                             __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
            *reinterpret_cast<u32x4*>(Xs + t * KP + k8) = o;
        }
        // (more pieces than the prefetch holds: several tokens of a long row;
        // loaded and stored the same way)
        if constexpr (TV > 1) {
            for (int q = tid + XPT * NT; q < npieces; q += NT) {
                const int t = q / (KP / 8), k8 = (q - t * (KP / 8)) * 8;
                u32x4 v = *reinterpret_cast<const u32x4*>(p.X + (int64_t)min(t, p.T - 1) * K + min(k8, K - 8));
                if (t >= p.T || k8 >= K) v = u32x4{0u, 0u, 0u, 0u};
                const u32x4 o = {__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                                 __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
                *reinterpret_cast<u32x4*>(Xs + t * KP + k8) = o;
            }
        }
    } else {
        for (int idx = tid; idx < TV * KP; idx += NT) {
            const int t = idx / KP, k = idx - t * KP;
            Xs[t * KP + xperm(k)] = (t < p.T && k < K) ? p.X[(int64_t)t * K + k] : (uint16_t)0;
        }
    }
    if constexpr (!DX) lds_barrier();
    // DX: the lane's x in the unpack order, and their sum
    u32x4 xd[4];
    float sx = 0.0f;
    if constexpr (DX) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const u32x4 v = xr[d];
            xd[d] = u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                          __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
            sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].x), one, sx, false);
            sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].y), one, sx, false);
            sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].z), one, sx, false);
            sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].w), one, sx, false);
        }
    }

    float acc[RPW][TV];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < TV; ++t) acc[r][t] = 0.0f;
    constexpr unsigned C64 = 0x64646464u;

    for (int c0 = 0; c0 < nch; c0 += 64 * UPR) {
        if (c0 > 0) load_batch(c0);
#pragma unroll
        for (int u = 0; u < UPR; ++u) {
            if (c0 + 64 * u >= nch) break;  // uniform across the wave
            const int c = c0 + 64 * u + lane;
            const int cs = min(c, nch - 1);  // lanes past the end: garbage, masked by s = 0
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const bool valid = row0 + r % LR < p.O && c < nch;
                const float sc = valid ? h2f(sh[r][u]) : 0.0f;
                const f16x2 zz = mg::magic_zero(zh[r][u]);
                // (DX: 1024 + q; the zero point comes off per chunk below)
                f16x2 qz[16];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const unsigned w = a[r][u][d];
                    const unsigned hi = (w >> 4) & 0x0f0f0f0fu, lo = w & 0x0f0f0f0fu;
                    if constexpr (DX) {
                        qz[4 * d + 0] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04010400u));
                        qz[4 * d + 1] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04030402u));
                        qz[4 * d + 2] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04010400u));
                        qz[4 * d + 3] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04030402u));
                    } else {
                        qz[4 * d + 0] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04010400u)) - zz;
                        qz[4 * d + 1] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04030402u)) - zz;
                        qz[4 * d + 2] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04010400u)) - zz;
                        qz[4 * d + 3] = bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04030402u)) - zz;
                    }
                }
#pragma unroll
                for (int t = 0; t < TV; ++t) {
                    const u32x4* xv = reinterpret_cast<const u32x4*>(Xs + t * KP + 32 * cs);
                    float dot = 0.0f;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const u32x4 x = DX ? xd[d] : xv[d];
                        dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.x), qz[4 * d + 0], dot, false);
                        dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.y), qz[4 * d + 1], dot, false);
                        dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.z), qz[4 * d + 2], dot, false);
                        dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.w), qz[4 * d + 3], dot, false);
                    }
                    if constexpr (DX) dot = fmaf(-static_cast<float>(zz[0]), sx, dot);
                    acc[r][t] = fmaf(sc, dot, acc[r][t]);
                }
            }
        }
    }
    // the wave's sums (a fixed butterfly, permlane swaps and DPP): every lane
    // ends with the totals
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < TV; ++t) acc[r][t] = wave_sum(acc[r][t]);
    // lane t (t < T) writes token t of every row
    if constexpr (SWIGLU) {
#pragma unroll
        for (int r = 0; r < LR; ++r) {
            const int row = row0 + r;
            if (row >= p.O || lane >= p.T || lane >= TV) continue;
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int t = 0; t < TV; ++t)
                if (t == lane) {
                    g = acc[r][t];
                    u = acc[r + LR][t];
                }
            p.Y[(int64_t)lane * p.O + row] = swiglu_h(f2h(g), f2h(u));
        }
        return;
    }
    // beta != 0: every old output of the lane is loaded (clamped indices)
    // before the first store, since a load issued after a store waits for it
    float old[RPW];
    if (p.beta != 0.0f) {
        const uint16_t* src = p.Y + (int64_t)min(lane, p.T - 1) * p.O;
#pragma unroll
        for (int r = 0; r < RPW; ++r) old[r] = h2f(src[min(row0 + r, p.O - 1)]);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + r;
        if (row >= p.O || lane >= p.T || lane >= TV) continue;
        float v = 0.0f;
#pragma unroll
        for (int t = 0; t < TV; ++t)
            if (t == lane) v = acc[r][t];
        float y = p.alpha * v;
        if (p.beta != 0.0f) y = fmaf(p.beta, old[r], y);
        p.Y[(int64_t)lane * p.O + row] = f2h(y);
    }
}

// One token on longer rows (65 to 512 chunks: K % 32 == 0, aligned W and X):
// the KS = ceil(nch / 64) waves of a workgroup share RPW rows and split K,
// wave w taking chunk 64 w + lane of every row, its x straight into
// registers and the zero point taken out per chunk as in DX; each wave sums
// its lanes (the fixed butterfly), then wave 0 adds the KS partials of each
// row in wave order.  X is read once per workgroup and never staged, and its
// permute and sum serve RPW rows.  Cold graph replays, us per call, against
// the row-per-wave GEMV with X staged in LDS: 2048 x 8192 (Llama-1B down)
// 5.48 -> 4.68, 4096 x 4096 5.13 -> 4.65, 11008 x 4096 8.60 -> 7.17, 4096 x
// 11008 9.32 -> 7.80, 14336 x 4096 9.88 -> 8.50, 8192 x 8192 12.05 -> 9.37,
// 2048 x 16384 20.70 -> 6.59; four rows per workgroup ahead of two and one
// (11008 x 4096: 7.24 / 8.05 / 10.39) wherever they still give two workgroups
// per CU.
template <int RPW>
__global__ void __launch_bounds__(512) w4a16_gemv_ks(GemvParams p) {
    __shared__ float part[8][RPW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KS = blockDim.x >> 6;
    const int nch = p.nch, K = p.K, G = p.G;
    const int row0 = blockIdx.x * RPW;
    const int c = wave * 64 + lane;
    const int cs = min(c, nch - 1);  // lanes past the end: garbage, masked by s = 0
    u32x4 xr[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) xr[d] = *reinterpret_cast<const u32x4*>(p.X + 32 * cs + 8 * d);
    u32x4 a[RPW];
    uint16_t sh[RPW], zh[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(row0 + r, p.O - 1);
        a[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.W + (int64_t)row * (K / 2) + 16 * cs));
        const int64_t gi = (int64_t)row * G + (cs >> 2);
        sh[r] = p.scale[gi];
        zh[r] = p.zero[gi];
    }
    // x in the unpack order (x0 x2)(x4 x6)(x1 x3)(x5 x7) per 8 k, and their sum
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    u32x4 xd[4];
    float sx = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const u32x4 v = xr[d];
        xd[d] = u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                      __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
        sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].x), one, sx, false);
        sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].y), one, sx, false);
        sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].z), one, sx, false);
        sx = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].w), one, sx, false);
    }
    constexpr unsigned C64 = 0x64646464u;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const bool valid = row0 + r < p.O && c < nch;
        const float sc = valid ? h2f(sh[r]) : 0.0f;
        const f16x2 zz = mg::magic_zero(zh[r]);
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const unsigned w = a[r][d];
            const unsigned hi = (w >> 4) & 0x0f0f0f0fu, lo = w & 0x0f0f0f0fu;
            dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].x), bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04010400u)),
                                         dot, false);
            dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].y), bitcast<f16x2>(__builtin_amdgcn_perm(C64, hi, 0x04030402u)),
                                         dot, false);
            dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].z), bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04010400u)),
                                         dot, false);
            dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(xd[d].w), bitcast<f16x2>(__builtin_amdgcn_perm(C64, lo, 0x04030402u)),
                                         dot, false);
        }
        dot = fmaf(-static_cast<float>(zz[0]), sx, dot);
        acc[r] = wave_sum(sc * dot);
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) part[wave][r] = acc[r];
    }
    __syncthreads();
    if (wave != 0 || lane >= RPW) return;
    float v = part[0][lane];
    for (int w = 1; w < KS; ++w) v += part[w][lane];
    const int row = row0 + lane;
    if (row >= p.O) return;
    float y = p.alpha * v;
    if (p.beta != 0.0f) y = fmaf(p.beta, h2f(p.Y[row]), y);
    p.Y[row] = f2h(y);
}

namespace {

constexpr size_t kMaxGemvLds = 150 * 1024;

// Rows per wave RPW and waves per workgroup: as many chunk loads per lane in
// flight as fit (8), then enough workgroups to cover every CU.
struct GemvShape {
    int rpw, upr, wpb;
};
// (wg_min: workgroups per CU the first halving aims for)
inline GemvShape gemv_shape(int rows, int nch, int cus, int wg_min = 1) {
    const int cpl = cdiv(nch, 64);
    GemvShape g{1, 8, 16};
    if (cpl >= 7) g = {1, 8, 16};
    else if (cpl >= 5) g = {1, 6, 16};
    else if (cpl >= 3) g = {2, 4, 16};
    else if (cpl == 2) g = {4, 2, 16};
    else g = {8, 1, 16};
    while (g.wpb > 4 && cdiv(rows, g.wpb * g.rpw) < wg_min * cus) g.wpb >>= 1;
    // fewer rows per wave, up to two workgroups per CU: the rows spread over
    // the CUs evenly (3072 rows at K = 2048: 768 workgroups, 3 per CU, rather
    // than 384, some CUs holding twice the rows of others); a lane never
    // loads more chunks per row than the row has
    const int target = 2 * cus;
    while (g.rpw > 1 && cdiv(rows, g.wpb * g.rpw) < target) { g.rpw >>= 1; g.upr <<= 1; }
    // (rounded up to an instantiated width: 1, 2, 4, 6, 8)
    if (g.upr > cpl) g.upr = cpl <= 2 ? cpl : cpl <= 4 ? 4 : cpl <= 6 ? 6 : 8;
    if (g.upr > 8) g.upr = 8;
    return g;
}

// DX (X straight into registers, no LDS) wherever it applies: one token, one
// aligned chunk per lane, aligned X (cold graph replays, us per call: Llama-1B
// decode QKV 3072 x 2048 3.62 -> 3.44, O 2048 x 2048 3.44 -> 3.36, gate/up +
// SwiGLU 2 x 8192 x 2048 6.80 -> 6.08; down 2048 x 8192, four chunks per lane,
// measured slower with X in registers, 5.31 -> 5.84, and keeps the LDS)
template <int TV, int RPW, int UPR, bool ALIGNED, bool SWIGLU = false>
clove_status_t run_gemv_shape(const GemvParams& p, int wpb, hipStream_t stream) {
    // (not with eight rows per wave: their weights and x do not fit the VGPRs)
    constexpr bool DXOK = TV == 1 && UPR == 1 && ALIGNED && RPW <= 4;
    const bool dx = DXOK && p.nch <= 64 && aligned16(p.X);
    const size_t lds = dx ? 0 : gemv_lds_bytes(TV, p.nch);
    wpb = min(wpb, w4_max_threads<TV, RPW, UPR, ALIGNED>() / 64);
    const dim3 grid(cdiv(p.O, wpb * (SWIGLU ? RPW / 2 : RPW)));
    auto k = dx ? w4a16_gemv<TV, RPW, UPR, ALIGNED, SWIGLU, DXOK> : w4a16_gemv<TV, RPW, UPR, ALIGNED, SWIGLU>;
    if (ensure_lds(reinterpret_cast<const void*>(k), (int)lds) != CLOVE_OK) return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, grid, dim3(wpb * 64), lds, stream, p);
    return check_launch();
}

// SwiGLU: gate / up pairs, so at least two weight rows per wave (the shape
// is chosen for the 2 O weight rows).  One token on rows of two or more chunks
// per lane: workgroups halved to two per CU (cold: 11008 x 4096 16.0 -> 14.7
// us, 14336 x 4096 19.7 -> 17.7, 4096 x 8192 11.9 -> 10.3; 2..4 tokens, whose
// lanes hold more registers, and the plain GEMV measured slower or no better
// with it: 14336 x 4096 T = 4 28.0 -> 36.1)
template <int TV>
clove_status_t run_gemv_swiglu(const GemvParams& p, bool aligned, int cus, hipStream_t stream) {
    const GemvShape g = gemv_shape(2 * p.O, p.nch, cus, TV == 1 && cdiv(p.nch, 64) >= 2 ? 2 : 1);
    // unaligned rows are assembled from byte loads (16 registers per chunk
    // until packed): one gate / up pair per wave and one chunk per lane at a
    // time, so that the variant needs no scratch
    if (!aligned) return run_gemv_shape<TV, 2, 1, false, true>(p, g.wpb, stream);
    // (a lane loads no more chunks per row than the row has: two-row waves
    // take 1, 2 or 4 chunk loads per row)
    if (g.rpw == 1) return run_gemv_shape<TV, 2, 4, true, true>(p, g.wpb, stream);
    if (g.rpw == 2) return g.upr <= 1   ? run_gemv_shape<TV, 2, 1, true, true>(p, g.wpb, stream)
                           : g.upr <= 2 ? run_gemv_shape<TV, 2, 2, true, true>(p, g.wpb, stream)
                                        : run_gemv_shape<TV, 2, 4, true, true>(p, g.wpb, stream);
    if (g.rpw == 4) return g.upr == 1 ? run_gemv_shape<TV, 4, 1, true, true>(p, g.wpb, stream)
                                      : run_gemv_shape<TV, 4, 2, true, true>(p, g.wpb, stream);
    return run_gemv_shape<TV, 8, 1, true, true>(p, g.wpb, stream);
}

// One token on rows of 65..512 aligned chunks: w4a16_gemv_ks, four rows per
// workgroup while that leaves two workgroups per CU, else two or one
template <int TV>
bool try_gemv_ks(const GemvParams& p, bool aligned, int cus, hipStream_t stream, clove_status_t* st) {
    const int ks = cdiv(p.nch, 64);
    if (TV != 1 || !aligned || !aligned16(p.X) || ks < 2 || ks > 8) return false;
    const int rpw = cdiv(p.O, 4) >= 2 * cus ? 4 : cdiv(p.O, 2) >= cus ? 2 : 1;
    const dim3 grid(cdiv(p.O, rpw)), block(64 * ks);
    if (rpw == 4) CLOVE_LAUNCH(w4a16_gemv_ks<4>, grid, block, 0, stream, p);
    else if (rpw == 2) CLOVE_LAUNCH(w4a16_gemv_ks<2>, grid, block, 0, stream, p);
    else CLOVE_LAUNCH(w4a16_gemv_ks<1>, grid, block, 0, stream, p);
    *st = check_launch();
    return true;
}

template <int TV>
clove_status_t run_gemv(const GemvParams& p, bool aligned, int cus, hipStream_t stream) {
    clove_status_t kst;
    if (try_gemv_ks<TV>(p, aligned, cus, stream, &kst)) return kst;
    GemvShape g = gemv_shape(p.O, p.nch, cus);
    // one token on rows of two or more chunks per lane: workgroups halved until
    // there are four per CU (rows of two chunks) or two (longer rows); cold:
    // 14336 x 4096 9.9 -> 9.1 us, 4096 x 14336 10.8 -> 10.4, 4096 x 11008 9.35 ->
    // 9.03, 11008 x 4096 8.0 -> 7.8, eight other weight shapes unchanged
    if (TV == 1 && cdiv(p.nch, 64) >= 2) {
        const int target = (cdiv(p.nch, 64) == 2 ? 4 : 2) * cus;
        while (g.wpb > 4 && cdiv(p.O, g.wpb * g.rpw) < target) g.wpb >>= 1;
    }
    // two to four tokens on rows of two or more chunks per lane: every
    // workgroup stages all of X in LDS, so workgroups grow (while at least one
    // per CU remains) until they hold 4 TV rows and the X copies stay within the
    // weight bytes (cold: 2048 x 8192 T = 2 6.9 -> 6.1 us, 2048 x 4096 T = 4
    // 6.2 -> 5.6; one-chunk rows and thinner grids measured slower with it)
    if (TV > 1 && cdiv(p.nch, 64) >= 2) {
        const int maxw = w4_max_threads<TV, 1, 1, true>() / 64;
        while (g.wpb * g.rpw < 4 * TV && g.wpb * 2 <= maxw && cdiv(p.O, 2 * g.wpb * g.rpw) >= cus) g.wpb <<= 1;
    }
    // (unaligned rows: one row per wave and one chunk per lane at a time, as
    // for the SwiGLU variant)
    if (!aligned) return run_gemv_shape<TV, 1, 1, false>(p, g.wpb, stream);
    // (rpw, upr) pairs keep rpw * upr <= 8 chunk loads per lane
    if (g.rpw == 1) {
        if (g.upr >= 8) return run_gemv_shape<TV, 1, 8, true>(p, g.wpb, stream);
        if (g.upr >= 6) return run_gemv_shape<TV, 1, 6, true>(p, g.wpb, stream);
        if (g.upr >= 4) return run_gemv_shape<TV, 1, 4, true>(p, g.wpb, stream);
        if (g.upr >= 2) return run_gemv_shape<TV, 1, 2, true>(p, g.wpb, stream);
        return run_gemv_shape<TV, 1, 1, true>(p, g.wpb, stream);
    }
    if (g.rpw == 2) return g.upr <= 1   ? run_gemv_shape<TV, 2, 1, true>(p, g.wpb, stream)
                           : g.upr <= 2 ? run_gemv_shape<TV, 2, 2, true>(p, g.wpb, stream)
                                        : run_gemv_shape<TV, 2, 4, true>(p, g.wpb, stream);
    if (g.rpw == 4) return g.upr == 1 ? run_gemv_shape<TV, 4, 1, true>(p, g.wpb, stream)
                                      : run_gemv_shape<TV, 4, 2, true>(p, g.wpb, stream);
    return run_gemv_shape<TV, 8, 1, true>(p, g.wpb, stream);
}

using mg::Tile;

template <class T, bool ALIGNED>
clove_status_t run_mfma(mg::Params p, int cus, hipStream_t stream) {
    using LA = mg::LoadF16Rows<T::BM, T::BK, T::NT, T::LDK, false, ALIGNED>;
    using LB = mg::LoadI4Rows<T::BN, T::BK, T::NT, T::LDK, true, mg::kI4Groupwise, ALIGNED>;
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
    CLOVE_LAUNCH((mg::mfma_gemm<T, LA, LB, mg::EpiAlphaBeta<ALIGNED>, mg::kFoldB>), dim3(tiles * p.nsplit),
                       dim3(T::NT), 0, stream, p);
    return check_launch();
}

}  // namespace
}  // namespace w4

clove_status_t launch_w4a16_swiglu(const W4A16Args& a, hipStream_t stream) {
    using namespace w4;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const int G = cdiv(a.K, 128);
    const int nch = cdiv(a.K, 32);
    const int tv = a.T <= 1 ? 1 : (a.T <= 2 ? 2 : 4);
    if (a.T <= 4 && gemv_lds_bytes(tv, nch) <= kMaxGemvLds) {
        GemvParams p{a.X, a.W, a.scale, a.zero, a.Y, a.T, a.O, a.K, G, nch, 1.0f, 0.0f};
        const bool aligned = aligned16(a.W) && (a.K % 32 == 0);
        if (tv == 1) return run_gemv_swiglu<1>(p, aligned, dev.num_cus, stream);
        if (tv == 2) return run_gemv_swiglu<2>(p, aligned, dev.num_cus, stream);
        return run_gemv_swiglu<4>(p, aligned, dev.num_cus, stream);
    }
    clove_status_t st2;
    if (try_i4w_w4a16_swiglu(a, dev.num_cus, stream, &st2)) return st2;
    // other shapes: gate into H, up into a library buffer, SwiGLU in place
    void* ubuf = nullptr;
    st = acquire_buffer(stream, kBufSwiglu, (size_t)a.T * a.O * 2, &ubuf);
    if (st != CLOVE_OK) return st;
    W4A16Args g = a, u = a;
    g.alpha = u.alpha = 1.0f;
    g.beta = u.beta = 0.0f;
    u.W = a.W + (size_t)a.O * (a.K / 2);
    u.scale = a.scale + (size_t)a.O * G;
    u.zero = a.zero + (size_t)a.O * G;
    u.Y = static_cast<uint16_t*>(ubuf);
    if ((st = launch_w4a16(g, stream)) != CLOVE_OK) return st;
    if ((st = launch_w4a16(u, stream)) != CLOVE_OK) return st;
    return launch_swiglu(a.Y, u.Y, a.Y, (int64_t)a.T * a.O, stream);
}

clove_status_t launch_w4a16(const W4A16Args& a, hipStream_t stream) {
    using namespace w4;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const int G = cdiv(a.K, 128);
    const int nch = cdiv(a.K, 32);
    const int tv = a.T <= 1 ? 1 : (a.T <= 2 ? 2 : 4);
    if (a.K > 0 && a.T >= 3 && a.T <= 4) {
        // (large weights: the streaming kernel, see try_i4w_w4a16)
        clove_status_t st2;
        if (try_i4w_w4a16(a, dev.num_cus, stream, &st2)) return st2;
    }
    if (a.K > 0 && a.T <= 4 && gemv_lds_bytes(tv, nch) <= kMaxGemvLds) {
        GemvParams p{a.X, a.W, a.scale, a.zero, a.Y, a.T, a.O, a.K, G, nch, a.alpha, a.beta};
        const bool aligned = aligned16(a.W) && (a.K % 32 == 0);
        if (tv == 1) return run_gemv<1>(p, aligned, dev.num_cus, stream);
        if (tv == 2) return run_gemv<2>(p, aligned, dev.num_cus, stream);
        return run_gemv<4>(p, aligned, dev.num_cus, stream);
    }
    if (a.K > 0) {
        clove_status_t st2;
        if (try_i4w_w4a16(a, dev.num_cus, stream, &st2)) return st2;
    }
    mg::Params p{};
    p.a = a.X;
    p.b = a.W; p.b_scale = a.scale; p.b_zero = a.zero;
    p.c = a.Y;
    p.M = a.T; p.N = a.O; p.K = a.K; p.G = G;
    p.alpha = a.alpha; p.beta = a.beta;
    const bool aligned = aligned16(a.X) && aligned16(a.W) && aligned16(a.Y) && (a.K % 32 == 0) &&
                         (a.O % 8 == 0);
    if (!aligned) return run_mfma<Tile<64, 64, 64, 2, 2>, false>(p, dev.num_cus, stream);
    return run_mfma<Tile<128, 128, 64, 2, 2>, true>(p, dev.num_cus, stream);
}

}  // namespace clove
