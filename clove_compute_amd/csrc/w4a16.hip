// W4A16 linear layer for gfx950: Y = alpha * X @ dequant(W)^T + beta * Y.
//
// X [T,K] fp16 activations, W_q [O, K/2] group-128 INT4 weights in gemm_int4's
// A layout (src/kernels/gemm_int4.cu:27-34: even k in the high nibble), scales
// and zeros [O, G].  It is the reference runtime's linear-layer call
// (src/runtime/inference.cu:139-194, beta = 1 residual at :165-168, :191-194)
// on INT4 weights.
//
//  * w4a16_gemv (T <= 4, decode) -- LPR lanes stream one weight row with
//    16-byte loads.  Per 32-k chunk and token:
//        sum_k x_k (q_k - z) = sum_k x_k (1024 + q_k) - (1024 + z) * sum_k x_k
//    where 1024 + q is the fp16 bit pattern 0x6400 | q, the first sum is
//    v_dot2_f32_f16 on (x pair, magic pair) and the chunk sums of x are staged
//    in LDS with X once per workgroup.  acc += scale * that, in fp32.
//  * larger T -- the shared MFMA GEMM (mfma_gemm.hpp): X rows as operand A,
//    W rows unpacked to the exact integers q - z as operand B; the per-group
//    fp32 partials are scaled by s[o,g] after each 128-wide group.
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

// LDS (dynamic): Xs [TV][32*nch] fp16 | Xsum [TV][nch] f32
__host__ __device__ inline size_t gemv_lds_bytes(int tv, int nch) {
    return (size_t)tv * ((size_t)32 * nch * 2 + (size_t)nch * 4);
}

template <int TV, int LPR, bool ALIGNED>
__global__ void __launch_bounds__(256) w4a16_gemv(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned lds[];
    constexpr int RPW = 256 / LPR;
    constexpr int UNR = 4;
    const int tid = threadIdx.x;
    const int nch = p.nch, K = p.K, G = p.G;
    const int KP = 32 * nch;
    uint16_t* Xs = reinterpret_cast<uint16_t*>(lds);
    float* Xsum = reinterpret_cast<float*>(Xs + TV * KP);

    const int row = blockIdx.x * RPW + tid / LPR;
    const int lr = tid % LPR;
    const bool row_ok = row < p.O;
    const uint8_t* wrow = p.W + (int64_t)row * (K / 2);

    unsigned a_cur[UNR][4];
    uint16_t s_cur[UNR], z_cur[UNR];
    auto load_batch = [&](int c0, unsigned (&a)[UNR][4], uint16_t (&s)[UNR], uint16_t (&z)[UNR]) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int c = c0 + u * LPR;
            const bool in = row_ok && c < nch;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (in) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + 16 * c));
                a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
            } else {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    unsigned w = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int byte = 16 * c + 4 * d + e;
                        const unsigned b = (in && 2 * byte < K) ? wrow[byte] : 0u;
                        w |= b << (8 * e);
                    }
                    a[u][d] = w;
                }
            }
            const int64_t gi = (int64_t)row * G + (c >> 2);
            s[u] = in ? p.scale[gi] : (uint16_t)0;
            z[u] = in ? p.zero[gi] : (uint16_t)0;
        }
    };
    load_batch(lr, a_cur, s_cur, z_cur);

    // ---- stage X (zero-padded to whole chunks) and its chunk sums ----
    for (int idx = tid; idx < TV * KP; idx += 256) {
        const int t = idx / KP, k = idx - t * KP;
        Xs[idx] = (t < p.T && k < K) ? p.X[(int64_t)t * K + k] : (uint16_t)0;
    }
    __syncthreads();
    for (int idx = tid; idx < TV * nch; idx += 256) {
        const int t = idx / nch, c = idx - t * nch;
        const uint16_t* xc = Xs + t * KP + 32 * c;
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) s += h2f(xc[e]);
        Xsum[idx] = s;
    }
    __syncthreads();

    float acc[TV];
#pragma unroll
    for (int t = 0; t < TV; ++t) acc[t] = 0.0f;

    for (int c0 = lr; c0 < nch; c0 += UNR * LPR) {
        unsigned a_nxt[UNR][4];
        uint16_t s_nxt[UNR], z_nxt[UNR];
        const bool more = c0 + UNR * LPR < nch;
        if (more) load_batch(c0 + UNR * LPR, a_nxt, s_nxt, z_nxt);
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int c = c0 + u * LPR;
            if (c >= nch) break;
            unsigned mg16[16];
#pragma unroll
            for (int d = 0; d < 4; ++d) mg::nibbles_to_magic(a_cur[u][d], &mg16[4 * d]);
            const float s = h2f(s_cur[u]);
            const float zoff = 1024.0f + rintf(h2f(z_cur[u]));
#pragma unroll
            for (int t = 0; t < TV; ++t) {
                const u32x4* xv = reinterpret_cast<const u32x4*>(Xs + t * KP + 32 * c);
                float dot = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const u32x4 x = xv[v];
                    dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.x), bitcast<f16x2>(mg16[4 * v + 0]), dot, false);
                    dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.y), bitcast<f16x2>(mg16[4 * v + 1]), dot, false);
                    dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.z), bitcast<f16x2>(mg16[4 * v + 2]), dot, false);
                    dot = __builtin_amdgcn_fdot2(bitcast<f16x2>(x.w), bitcast<f16x2>(mg16[4 * v + 3]), dot, false);
                }
                const float P = fmaf(-zoff, Xsum[t * nch + c], dot);
                acc[t] = fmaf(s, P, acc[t]);
            }
        }
        if (more) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
#pragma unroll
                for (int d = 0; d < 4; ++d) a_cur[u][d] = a_nxt[u][d];
                s_cur[u] = s_nxt[u];
                z_cur[u] = z_nxt[u];
            }
        }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1)
#pragma unroll
        for (int t = 0; t < TV; ++t) acc[t] += __shfl_xor(acc[t], off);
    if (row_ok && lr < TV && lr < p.T) {
        // lane t writes token t's output
        float v = 0.0f;
#pragma unroll
        for (int t = 0; t < TV; ++t)
            if (t == lr) v = acc[t];
        uint16_t* dst = p.Y + (int64_t)lr * p.O + row;
        float r = p.alpha * v;
        if (p.beta != 0.0f) r = fmaf(p.beta, h2f(*dst), r);
        *dst = f2h(r);
    }
}

namespace {

constexpr size_t kMaxGemvLds = 150 * 1024;

template <int TV>
clove_status_t run_gemv(const GemvParams& p, bool aligned, hipStream_t stream) {
    constexpr int LPR = 32;
    const size_t lds = gemv_lds_bytes(TV, p.nch);
    const dim3 grid(cdiv(p.O, 256 / LPR));
    auto k = aligned ? w4a16_gemv<TV, LPR, true> : w4a16_gemv<TV, LPR, false>;
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return CLOVE_ERR_LAUNCH;
    hipLaunchKernelGGL(k, grid, dim3(256), lds, stream, p);
    return check_launch();
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
    hipLaunchKernelGGL((mg::mfma_gemm<T, LA, LB, mg::EpiAlphaBeta<ALIGNED>, mg::kFoldB>), dim3(tiles * p.nsplit),
                       dim3(T::NT), 0, stream, p);
    return check_launch();
}

}  // namespace
}  // namespace w4

clove_status_t launch_w4a16(const W4A16Args& a, hipStream_t stream) {
    using namespace w4;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    const int G = cdiv(a.K, 128);
    const int nch = cdiv(a.K, 32);
    const int tv = a.T <= 1 ? 1 : (a.T <= 2 ? 2 : 4);
    if (a.K > 0 && a.T <= 4 && gemv_lds_bytes(tv, nch) <= kMaxGemvLds) {
        GemvParams p{a.X, a.W, a.scale, a.zero, a.Y, a.T, a.O, a.K, G, nch, a.alpha, a.beta};
        const bool aligned = aligned16(a.W) && (a.K % 32 == 0);
        if (tv == 1) return run_gemv<1>(p, aligned, stream);
        if (tv == 2) return run_gemv<2>(p, aligned, stream);
        return run_gemv<4>(p, aligned, stream);
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
