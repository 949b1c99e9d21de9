// Generic LDS-tiled fp16 MFMA GEMM for gfx950 with pluggable tile loaders.
//
//   C[M,N] = epilogue( sum_k A[m,k] * B[k,n] )      fp32 accumulation
//
// Both operands are staged in LDS as fp16, K-contiguous per row (sA[m][k],
// sB[n][k]), so every MFMA fragment is one ds_read_b128.  A loader turns one
// (rows x BK) slice of its operand into that layout: fp16 rows are copied,
// fp16 N-contiguous B is transposed in registers, packed INT4 is unpacked to
// the exact small integers q - zero (or q - 8 for the reference-literal mode).
//
// INT4 group scales are not folded into the operands (that would round
// (q - z) * s to fp16).  With FOLD the kernel keeps per-group fp32 partials
// P_g (exact integers for INT4 x INT4) and after each 128-wide K group adds
// scale * P_g to the accumulator, scale = sA[m,g] * sB[g,n] (kFoldAB) or
// sB[n,g] (kFoldB); the loaders stage the group's scales in LDS.
//
// Wave tiling: WGM x WGN waves, each owning (BM/WGM) x (BN/WGN) outputs as a
// grid of 32x32 v_mfma_f32_32x32x16_f16 tiles.  The MFMA "A" operand is the B
// fragment (rows = n) and the MFMA "B" operand is the A fragment (cols = m), so
// each lane ends up holding 4 consecutive n of one output row: 8-byte stores.
//
// K loop: two LDS stages; the next K tile's global loads are issued before the
// current tile's MFMAs and written to the other stage afterwards (one barrier
// per K tile).  Optional split-K: each workgroup publishes its fp32 partial
// tile; the last to arrive sums all partials in split order (deterministic)
// and runs the epilogue.
#pragma once

#include "common.hpp"

namespace clove {
namespace mg {

using namespace hw;

struct Params {
    const void* a;             // operand A (rows m)
    const uint16_t* a_scale;   // INT4: [M, G] fp16
    const uint16_t* a_zero;
    const void* b;             // operand B
    const uint16_t* b_scale;   // INT4 rows: [N, G]; INT4 cols: [G, N]
    const uint16_t* b_zero;
    uint16_t* c;
    int M, N, K;
    int G;                     // ceil(K / 128)
    int ldb_bytes;             // INT4 cols: bytes per K row of B
    int b_cols_valid;          // INT4 cols: columns >= this read as zero
    float alpha, beta;
    int64_t strideA, strideB, strideC;  // between batches, in units of the element (bytes for INT4)
    int tiles_m, tiles_n;
    int nsplit, k_per_split;
    float* ws;
    unsigned* counters;
};

enum I4Mode { kI4Groupwise = 0, kI4Literal = 1 };

__device__ __forceinline__ f16x8 lds_read_f16x8(const uint16_t* p) {
    return bitcast<f16x8>(*reinterpret_cast<const u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Loader: fp16 rows [R, K] (K-contiguous) -> lds[row][k]
// ---------------------------------------------------------------------------
template <int ROWS, int BK, int NT, int LDK, bool IS_B, bool ALIGNED>
struct LoadF16Rows {
    static constexpr int CH = ROWS * BK / 8;
    static constexpr int L = (CH + NT - 1) / NT;
    unsigned r[L][4];

    __device__ __forceinline__ void load(const Params& p, int batch, int r0, int k0, int kend,
                                         int tid) {
        const uint16_t* base = static_cast<const uint16_t*>(IS_B ? p.b : p.a) +
                               batch * (IS_B ? p.strideB : p.strideA);
        const int R = IS_B ? p.N : p.M;
        const int K = p.K;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int c = tid + i * NT;
            const int row = c / (BK / 8);
            const int kc = (c % (BK / 8)) * 8;
            const int gr = r0 + row;
            const int gk = k0 + kc;
            const bool in = (CH % NT == 0 || c < CH) && gr < R;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (in && gk < kend) v = *reinterpret_cast<const u32x4*>(base + (int64_t)gr * K + gk);
                r[i][0] = v.x; r[i][1] = v.y; r[i][2] = v.z; r[i][3] = v.w;
            } else {
                uint16_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    h[e] = (in && gk + e < kend) ? base[(int64_t)gr * K + gk + e] : (uint16_t)0;
#pragma unroll
                for (int d = 0; d < 4; ++d) r[i][d] = h[2 * d] | ((unsigned)h[2 * d + 1] << 16);
            }
        }
    }

    __device__ __forceinline__ void store(const Params&, uint16_t* lds, float*, int, int tid) const {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int c = tid + i * NT;
            if (CH % NT != 0 && c >= CH) continue;
            const int row = c / (BK / 8);
            const int kc = (c % (BK / 8)) * 8;
            u32x4 v = {r[i][0], r[i][1], r[i][2], r[i][3]};
            *reinterpret_cast<u32x4*>(&lds[row * LDK + kc]) = v;
        }
    }
};

// ---------------------------------------------------------------------------
// Loader: fp16 B [K, N] (N-contiguous) -> lds[n][k].  Each thread loads a
// KR x 8 block (KR rows of K, 16 bytes each) and transposes it in registers.
// ---------------------------------------------------------------------------
template <int COLS, int BK, int NT, int LDK, bool ALIGNED>
struct LoadF16Cols {
    static constexpr int KR = (((BK / 8) * (COLS / 8)) % NT == 0) ? 8
                              : (((BK / 4) * (COLS / 8)) % NT == 0) ? 4 : 2;
    static constexpr int BLOCKS = (BK / KR) * (COLS / 8);
    static constexpr int L = (BLOCKS + NT - 1) / NT;
    unsigned r[L][KR][4];

    __device__ __forceinline__ void load(const Params& p, int batch, int n0, int k0, int kend,
                                         int tid) {
        const uint16_t* B = static_cast<const uint16_t*>(p.b) + batch * p.strideB;
        const int N = p.N;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int b = tid + i * NT;
            const bool bin = BLOCKS % NT == 0 || b < BLOCKS;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
            const int gn = n0 + nb * 8;
#pragma unroll
            for (int rr = 0; rr < KR; ++rr) {
                const int gk = k0 + kb * KR + rr;
                if constexpr (ALIGNED) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (bin && gk < kend && gn < N)
                        v = *reinterpret_cast<const u32x4*>(B + (int64_t)gk * N + gn);
                    r[i][rr][0] = v.x; r[i][rr][1] = v.y; r[i][rr][2] = v.z; r[i][rr][3] = v.w;
                } else {
                    uint16_t h[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        h[e] = (bin && gk < kend && gn + e < N) ? B[(int64_t)gk * N + gn + e]
                                                                : (uint16_t)0;
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        r[i][rr][d] = h[2 * d] | ((unsigned)h[2 * d + 1] << 16);
                }
            }
        }
    }

    __device__ __forceinline__ void store(const Params&, uint16_t* lds, float*, int, int tid) const {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int b = tid + i * NT;
            if (BLOCKS % NT != 0 && b >= BLOCKS) continue;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                unsigned w[KR / 2];
#pragma unroll
                for (int j = 0; j < KR / 2; ++j) {
                    const unsigned lo = r[i][2 * j][c >> 1];
                    const unsigned hi = r[i][2 * j + 1][c >> 1];
                    w[j] = (c & 1) ? __builtin_amdgcn_perm(hi, lo, 0x07060302u)
                                   : __builtin_amdgcn_perm(hi, lo, 0x05040100u);
                }
                uint16_t* dst = &lds[(nb * 8 + c) * LDK + kb * KR];
                if constexpr (KR == 8) {
                    *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
                } else if constexpr (KR == 4) {
                    *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
                } else {
                    *reinterpret_cast<unsigned*>(dst) = w[0];
                }
            }
        }
    }
};

// ---------------------------------------------------------------------------
// INT4 unpacking.  A byte holds an even-k nibble (high) and the following
// odd-k nibble (low).  0x6400 | q is the fp16 value 1024 + q, so
// (1024 + q) - (1024 + z) is q - z exactly (one packed fp16 subtract).
// ---------------------------------------------------------------------------
// 8 nibbles of one dword (k order 0..7) -> 4 half2 holding 1024 + q, in k order
__device__ __forceinline__ void nibbles_to_magic(unsigned w, unsigned out[4]) {
    const unsigned hi = (w >> 4) & 0x0f0f0f0fu;  // k = 0,2,4,6
    const unsigned lo = w & 0x0f0f0f0fu;         // k = 1,3,5,7
    out[0] = __builtin_amdgcn_perm(lo, hi, 0x0c040c00u) | 0x64006400u;
    out[1] = __builtin_amdgcn_perm(lo, hi, 0x0c050c01u) | 0x64006400u;
    out[2] = __builtin_amdgcn_perm(lo, hi, 0x0c060c02u) | 0x64006400u;
    out[3] = __builtin_amdgcn_perm(lo, hi, 0x0c070c03u) | 0x64006400u;
}

// half2 (1024+q) -> q - z  (zz = 1024 + z; literal mode passes z = 8)
__device__ __forceinline__ unsigned magic_minus(unsigned magic, f16x2 zz) {
    return bitcast<unsigned>(bitcast<f16x2>(magic) - zz);
}

// zero point (fp16 bits) -> 1024 + rint(z) as half2 (the magic-domain offset)
__device__ __forceinline__ f16x2 magic_zero(uint16_t zbits) {
    const float z = rintf(h2f(zbits));
    const _Float16 m = static_cast<_Float16>(1024.0f + z);
    return f16x2{m, m};
}

// ---------------------------------------------------------------------------
// Loader: packed INT4 rows [R, K/2] (K-contiguous; gemm_int4's A, W4A16's W)
// -> fp16 lds[row][k] = q - z (exact).  16-byte chunks (32 k); BK divides the
// 128-wide group, so a chunk has one scale/zero.  The row's group scale goes
// to sc[row] (as fp32) for the fold.
// ---------------------------------------------------------------------------
template <int ROWS, int BK, int NT, int LDK, bool IS_B, int MODE, bool ALIGNED>
struct LoadI4Rows {
    static_assert(BK % 32 == 0 && 128 % BK == 0, "K tile must divide the group");
    static constexpr int CPR = BK / 32;
    static constexpr int CH = ROWS * CPR;
    static constexpr int L = (CH + NT - 1) / NT;
    unsigned q[L][4];
    uint16_t s[L], z[L];
    int kv[L];  // valid k values in the chunk (0..32)

    __device__ __forceinline__ void load(const Params& p, int batch, int r0, int k0, int kend,
                                         int tid) {
        const uint8_t* base = static_cast<const uint8_t*>(IS_B ? p.b : p.a) +
                              batch * (IS_B ? p.strideB : p.strideA);
        const uint16_t* sc = IS_B ? p.b_scale : p.a_scale;
        const uint16_t* zp = IS_B ? p.b_zero : p.a_zero;
        const int R = IS_B ? p.N : p.M;
        const int64_t rowb = p.K / 2;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int c = tid + i * NT;
            const int row = c / CPR;
            const int kc = (c % CPR) * 32;
            const int gr = r0 + row;
            const int gk = k0 + kc;
            const bool in = (CH % NT == 0 || c < CH) && gr < R && gk < kend;
            kv[i] = in ? min(32, kend - gk) : 0;
            const uint8_t* src = base + gr * rowb + gk / 2;
            if constexpr (ALIGNED) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (in) v = *reinterpret_cast<const u32x4*>(src);
                q[i][0] = v.x; q[i][1] = v.y; q[i][2] = v.z; q[i][3] = v.w;
            } else {
                unsigned by[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) by[j] = (in && gk + 2 * j < kend) ? src[j] : 0u;
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    q[i][d] = by[4 * d] | (by[4 * d + 1] << 8) | (by[4 * d + 2] << 16) | (by[4 * d + 3] << 24);
            }
            if constexpr (MODE == kI4Groupwise) {
                // rows past R still publish a (zero) scale; gk past kend keeps the group's
                const bool rin = (CH % NT == 0 || c < CH) && gr < R;
                const int64_t gi = (int64_t)gr * p.G + min(gk, p.K - 1) / 128;
                s[i] = rin ? sc[gi] : (uint16_t)0;
                z[i] = in ? zp[gi] : (uint16_t)0;
            }
        }
    }

    __device__ __forceinline__ void store(const Params&, uint16_t* lds, float* scl, int,
                                          int tid) const {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int c = tid + i * NT;
            if (CH % NT != 0 && c >= CH) continue;
            const int row = c / CPR;
            const int kc = (c % CPR) * 32;
            f16x2 zz;
            if constexpr (MODE == kI4Groupwise) {
                zz = magic_zero(z[i]);
                if (kc == 0) scl[row] = h2f(s[i]);
            } else {
                zz = f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
            }
            unsigned out[16];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                unsigned m4[4];
                nibbles_to_magic(q[i][d], m4);
#pragma unroll
                for (int e = 0; e < 4; ++e) out[4 * d + e] = magic_minus(m4[e], zz);
            }
            if (kv[i] < 32) {  // ragged K tail or out-of-range chunk: exact zeros
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    if (2 * e >= kv[i]) out[e] = 0u;
                    else if (2 * e + 1 >= kv[i]) out[e] &= 0xffffu;
                }
            }
            uint16_t* dst = &lds[row * LDK + kc];
#pragma unroll
            for (int v = 0; v < 4; ++v)
                *reinterpret_cast<u32x4*>(dst + 8 * v) =
                    u32x4{out[4 * v], out[4 * v + 1], out[4 * v + 2], out[4 * v + 3]};
        }
    }
};

// ---------------------------------------------------------------------------
// Loader: packed INT4 B [K, ldb_bytes] (two columns per byte, even n high;
// gemm_int4's B) with per-(group, column) scale/zero -> fp16 lds[n][k].  Each
// thread takes a KR x 16 block (KR rows of 8 bytes) and transposes it.
// ---------------------------------------------------------------------------
template <int COLS, int BK, int NT, int LDK, int MODE, bool ALIGNED>
struct LoadI4Cols {
    static constexpr int KR = (((BK / 4) * (COLS / 16)) % NT == 0 && (BK / 4) * (COLS / 16) >= NT) ? 4
                              : (((BK / 2) * (COLS / 16)) >= NT) ? 2 : 1;
    static constexpr int BLOCKS = (BK / KR) * (COLS / 16);
    static constexpr int L = (BLOCKS + NT - 1) / NT;
    unsigned q[L][KR][2];
    int nvalid[L];  // valid columns in the block (0..16)
    int kvalid[L];  // valid k rows in the block (0..KR)
    int gk0[L];

    __device__ __forceinline__ void load(const Params& p, int /*batch*/, int n0, int k0, int kend,
                                         int tid) {
        const uint8_t* B = static_cast<const uint8_t*>(p.b);
        const int ld = p.ldb_bytes;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int b = tid + i * NT;
            const bool bin = BLOCKS % NT == 0 || b < BLOCKS;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
            const int gn = n0 + nb * 16;
            const int gk = k0 + kb * KR;
            nvalid[i] = bin ? max(0, min(16, p.b_cols_valid - gn)) : 0;
            kvalid[i] = bin ? max(0, min(KR, kend - gk)) : 0;
            gk0[i] = gk;
#pragma unroll
            for (int rr = 0; rr < KR; ++rr) {
                const uint8_t* src = B + (int64_t)(gk + rr) * ld + gn / 2;
                const bool rin = rr < kvalid[i] && nvalid[i] > 0;
                if constexpr (ALIGNED) {
                    u32x2 v = {0u, 0u};
                    if (rin) v = *reinterpret_cast<const u32x2*>(src);
                    q[i][rr][0] = v.x; q[i][rr][1] = v.y;
                } else {
                    unsigned by[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) by[j] = (rin && 2 * j < nvalid[i]) ? src[j] : 0u;
                    q[i][rr][0] = by[0] | (by[1] << 8) | (by[2] << 16) | (by[3] << 24);
                    q[i][rr][1] = by[4] | (by[5] << 8) | (by[6] << 16) | (by[7] << 24);
                }
            }
        }
    }

    __device__ __forceinline__ void store(const Params& p, uint16_t* lds, float* scl, int n0,
                                          int tid) const {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int b = tid + i * NT;
            if (BLOCKS % NT != 0 && b >= BLOCKS) continue;
            const int kb = b % (BK / KR);
            const int nb = b / (BK / KR);
            const int gn = n0 + nb * 16;
            const int g = min(gk0[i], p.K - 1) / 128;
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                // column c of the block: nibble (c & 1 ? low : high) of byte c/2
                f16x2 zz;
                const bool cin = c < nvalid[i];
                if constexpr (MODE == kI4Groupwise) {
                    const int64_t gi = (int64_t)g * p.N + gn + c;
                    zz = magic_zero(cin ? p.b_zero[gi] : (uint16_t)0);
                    if (kb == 0) scl[nb * 16 + c] = cin ? h2f(p.b_scale[gi]) : 0.0f;
                } else {
                    zz = f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
                }
                const int word = (c >> 1) >> 2;
                const int shift = ((c >> 1) & 3) * 8 + ((c & 1) ? 0 : 4);
                uint16_t h[KR];
#pragma unroll
                for (int rr = 0; rr < KR; ++rr) {
                    const unsigned nib = (q[i][rr][word] >> shift) & 0xfu;
                    const unsigned magic = 0x6400u | nib;
                    const unsigned v = magic_minus(magic | (magic << 16), zz) & 0xffffu;
                    h[rr] = (cin && rr < kvalid[i]) ? (uint16_t)v : (uint16_t)0;
                }
                uint16_t* dst = &lds[(nb * 16 + c) * LDK + kb * KR];
                if constexpr (KR == 4) {
                    *reinterpret_cast<u32x2*>(dst) = u32x2{h[0] | ((unsigned)h[1] << 16),
                                                           h[2] | ((unsigned)h[3] << 16)};
                } else if constexpr (KR == 2) {
                    *reinterpret_cast<unsigned*>(dst) = h[0] | ((unsigned)h[1] << 16);
                } else {
                    dst[0] = h[0];
                }
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Epilogues: called with 4 consecutive columns gn..gn+3 of row gm.
// ---------------------------------------------------------------------------
// Each epilogue first loads what it reads (load, for every run of the tile,
// before any store: a load issued after a store to memory the compiler cannot
// tell apart waits for it, one round trip per run), then stores (apply).
template <bool ALIGNED>
struct EpiAlphaBeta {
    struct Pre {
        uint16_t old[4];
    };
    __device__ __forceinline__ static void load(const Params& p, const uint16_t* C, int gm, int gn, Pre& pre) {
        if (p.beta == 0.0f) return;
        const int N = p.N;
        const int64_t row = (int64_t)min(gm, p.M - 1) * N;
        if constexpr (ALIGNED) {
            const u32x2 c = *reinterpret_cast<const u32x2*>(C + row + min(gn, N - 4));
            pre.old[0] = (uint16_t)(c.x & 0xffffu);
            pre.old[1] = (uint16_t)(c.x >> 16);
            pre.old[2] = (uint16_t)(c.y & 0xffffu);
            pre.old[3] = (uint16_t)(c.y >> 16);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) pre.old[e] = C[row + min(gn + e, N - 1)];
        }
    }
    __device__ __forceinline__ static void apply(const Params& p, uint16_t* C, int gm, int gn,
                                                 const float acc[4], const Pre& pre) {
        const int N = p.N;
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[e] = p.alpha * acc[e];
            if (p.beta != 0.0f) r[e] = fmaf(p.beta, h2f(pre.old[e]), r[e]);
        }
        uint16_t* dst = C + (int64_t)gm * N + gn;
        if constexpr (ALIGNED) {
            if (gn >= N) return;
            *reinterpret_cast<u32x2*>(dst) = u32x2{pack2h(r[0], r[1]), pack2h(r[2], r[3])};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (gn + e < N) dst[e] = f2h(r[e]);
        }
    }
};

// The reference kernel's epilogue (src/kernels/gemm_int4.cu:185-190): the whole
// sum times the last group's scales, (acc * a_s) * b_s, rounded once to fp16.
struct EpiI4Literal {
    struct Pre {
        float a_s, b_s[4];
    };
    __device__ __forceinline__ static void load(const Params& p, const uint16_t*, int gm, int gn, Pre& pre) {
        const int g = p.G - 1;
        pre.a_s = h2f(p.a_scale[(int64_t)min(gm, p.M - 1) * p.G + g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) pre.b_s[e] = h2f(p.b_scale[(int64_t)g * p.N + min(gn + e, p.N - 1)]);
    }
    __device__ __forceinline__ static void apply(const Params& p, uint16_t* C, int gm, int gn,
                                                 const float acc[4], const Pre& pre) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int n = gn + e;
            if (n < p.N) C[(int64_t)gm * p.N + n] = f2h((acc[e] * pre.a_s) * pre.b_s[e]);
        }
    }
};

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
struct TileCoord {
    int batch, tm, tn, split;
};

// Workgroup id -> tile.  Workgroups go to the 8 XCDs round-robin; when the
// grid divides by 8 the id is permuted so each XCD owns a contiguous range of
// logical tiles, walked in groups of 8 tile-rows, so one XCD's workgroups share
// A and B panels in its L2.
__device__ __forceinline__ TileCoord decode_tile(const Params& p) {
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    TileCoord t;
    t.split = bid % p.nsplit;
    int tile = bid / p.nsplit;
    const int per_batch = p.tiles_m * p.tiles_n;
    t.batch = tile / per_batch;
    tile -= t.batch * per_batch;
    constexpr int GM = 8;
    const int group = tile / (GM * p.tiles_n);
    const int first_m = group * GM;
    const int gm = min(p.tiles_m - first_m, GM);
    const int in_group = tile - group * GM * p.tiles_n;
    t.tm = first_m + in_group % gm;
    t.tn = in_group / gm;
    return t;
}

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int NT = WGM * WGN * 64;
    static constexpr int LDK = BK + 8;  // 16-byte pad: conflict-free ds_read_b128 fragments
};

enum Fold { kFoldNone = 0, kFoldB = 1, kFoldAB = 2 };

template <class T, class LA, class LB, class EPI, int FOLD = kFoldNone, bool SPLITK = true>
__global__ void __launch_bounds__(T::NT) mfma_gemm(Params p) {
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, NT = T::NT, LDK = T::LDK;
    constexpr int WTM = BM / T::WGM;
    constexpr int WTN = BN / T::WGN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && BK % 16 == 0, "tile shape");
    static_assert(FOLD == kFoldNone || 128 % BK == 0, "fold needs K tiles inside one group");
    constexpr int SCA = FOLD == kFoldAB ? BM : 1;
    constexpr int SCB = FOLD != kFoldNone ? BN : 1;

    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) float sScA[2][SCA];
    __shared__ __attribute__((aligned(16))) float sScB[2][SCB];
    __shared__ int s_last;

    const TileCoord tc = decode_tile(p);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / T::WGN;
    const int wn = wave % T::WGN;
    const int m0 = tc.tm * BM;
    const int n0 = tc.tn * BN;
    const int kbeg = tc.split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int ktiles = kend > kbeg ? cdiv(kend - kbeg, BK) : 0;

    LA la;
    LB lb;
    auto stage_store = [&](int st) {
        la.store(p, sA[st], sScA[st], m0, tid);
        lb.store(p, sB[st], sScB[st], n0, tid);
    };

    f32x16 acc[FN][FM];
    f32x16 part[FOLD != kFoldNone ? FN : 1][FOLD != kFoldNone ? FM : 1];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if constexpr (FOLD != kFoldNone) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) part[i][j][r] = 0.0f;
    }

    if (ktiles > 0) {
        la.load(p, tc.batch, m0, kbeg, kend, tid);
        lb.load(p, tc.batch, n0, kbeg, kend, tid);
        stage_store(0);
        __syncthreads();
    }
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 8;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) {
            la.load(p, tc.batch, m0, kbeg + (kt + 1) * BK, kend, tid);
            lb.load(p, tc.batch, n0, kbeg + (kt + 1) * BK, kend, tid);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            f16x8 bf[FN], af[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i)
                bf[i] = lds_read_f16x8(&sB[st][(wn * WTN + i * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int j = 0; j < FM; ++j)
                af[j] = lds_read_f16x8(&sA[st][(wm * WTM + j * 32 + lrow) * LDK + kk + lk]);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    if constexpr (FOLD != kFoldNone)
                        part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], part[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[i], af[j], acc[i][j], 0, 0, 0);
                }
        }
        if constexpr (FOLD != kFoldNone) {
            // end of a 128-wide group (or of this split's K range): acc += scale * P_g
            const int knext = kbeg + (kt + 1) * BK;
            if ((knext & 127) == 0 || !more) {
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    const f32x4* sbv = reinterpret_cast<const f32x4*>(
                        &sScB[st][wn * WTN + i * 32 + (lane >> 5) * 4]);
                    f32x4 sb4[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) sb4[q] = sbv[2 * q];  // columns 8q .. 8q+3
#pragma unroll
                    for (int j = 0; j < FM; ++j) {
                        const float sa = FOLD == kFoldAB ? sScA[st][wm * WTM + j * 32 + lrow] : 1.0f;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const float sc = FOLD == kFoldAB ? sa * sb4[r >> 2][r & 3] : sb4[r >> 2][r & 3];
                            acc[i][j][r] = fmaf(sc, part[i][j][r], acc[i][j][r]);
                            part[i][j][r] = 0.0f;
                        }
                    }
                }
            }
        }
        if (more) stage_store(st ^ 1);
        __syncthreads();
    }

    if (SPLITK && p.nsplit > 1) {
        constexpr int NC = FN * FM * 4;  // f32x4 chunks per thread
        const int tile_id = (tc.batch * p.tiles_m + tc.tm) * p.tiles_n + tc.tn;
        float* slabs = p.ws + (int64_t)tile_id * p.nsplit * (BM * BN);
        f32x4 v[NC];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[(i * FM + j) * 4 + q] = f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                                    acc[i][j][4 * q + 3]};
        splitk_publish<NC, NT>(slabs + (int64_t)tc.split * (BM * BN), tid, v);
        if (!splitk_arrive_is_last(&p.counters[tile_id], (unsigned)p.nsplit, &s_last)) return;
        splitk_reduce<NC, NT, false>(slabs, p.nsplit, tc.split, tid, v);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = v[(i * FM + j) * 4 + q][e];
    }

    uint16_t* C = p.c + tc.batch * p.strideC;
    typename EPI::Pre pre[FN][FM][4];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                EPI::load(p, C, m0 + wm * WTM + j * 32 + lrow, n0 + wn * WTN + i * 32 + q * 8 + (lane >> 5) * 4,
                          pre[i][j][q]);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int gm = m0 + wm * WTM + j * 32 + lrow;
            if (gm >= p.M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int gn = n0 + wn * WTN + i * 32 + q * 8 + (lane >> 5) * 4;
                const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                    acc[i][j][4 * q + 3]};
                EPI::apply(p, C, gm, gn, v, pre[i][j][q]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
struct SplitPlan {
    int nsplit;
    int k_per_split;
};

// Split K only when the tile grid leaves CUs idle (tiles < num_cus): then
// about `target` workgroups run, each split keeping >= min_ktiles K tiles of
// width bk.
inline SplitPlan plan_split(int tiles, int K, int bk, int num_cus, int target, int min_ktiles) {
    SplitPlan sp{1, cdiv(K > 0 ? K : 1, bk) * bk};
    if (K <= 0 || tiles >= num_cus) return sp;
    const int ktiles = cdiv(K, bk);
    const int want = cdiv(target, tiles);
    const int maxs = max(1, ktiles / min_ktiles);
    const int ns = min(want, maxs);
    if (ns <= 1) return sp;
    const int kps = cdiv(ktiles, ns) * bk;
    sp.nsplit = cdiv(K, kps);
    sp.k_per_split = kps;
    return sp;
}

}  // namespace mg
}  // namespace clove
