// Host side of the INT4-weight MFMA GEMM (i4w_gemm.hpp): tile configuration,
// split-K plan, scratch, and the B transpose of group-wise INT4.
#include "dispatch.hpp"
#include "i4w_gemm.hpp"
#include "i4w_stream.hpp"

namespace clove {
namespace {

using namespace i4w;

// (WR, WC, FW, FX, stages): waves along weight rows x along X rows, 32x32
// tiles per wave in each direction
using CfgBig = Cfg<4, 1, 2, 4, 3>;  // 256 x 128, 4 waves of 64 x 128
// 128 x 64, one stage ahead (50 KB LDS: two workgroups per CU).  The
// prefill GEMMs are bound by the VALU and MFMA issue, not by their loads: a
// second stage in flight only made every workgroup's first stage wait behind
// a larger burst of the grid's prologue loads (W4A16 Llama-1B layer T = 512
// 125.6 -> 122.9 us, fused 114.9 -> 111.1 us against three stages)
using CfgC64 = Cfg<4, 1, 1, 2, 2>;
using CfgC32 = Cfg<2, 1, 1, 1, 4>;  // 64 x 32, 2 waves (several workgroups per CU)
// 256 x 64 (four waves of 64 x 64), one stage ahead (70 KB LDS: two workgroups
// per CU): the fused gate/up + SwiGLU from 512 X rows up, where each wave's two
// weight blocks (a gate and an up block per 32 outputs) share every X
// fragment it reads.  Measured against 128 x 64 / 256 x 128 on the Llama-1B
// and -7B MLPs (I x K = 8192 x 2048, 11008 x 4096; graph replays, cold
// weights), T = 512 (alternating blocks): 47.0-48.0 -> 45.0-45.2 and
// 119.3-119.8 -> 116.6-117.2 us, T = 1024: 94.8 -> 85.9 and 224.6 -> 217.2,
// T = 2048: 184.2 -> 166.2 and 470.8 -> 420.1; at T <= 256 it loses (T = 64:
// 14.6 -> 19.3)
using CfgS64 = Cfg<4, 1, 2, 2, 2>;
// 256 x 128 with eight waves of 64 x 64 (two per SIMD), one stage ahead
// (100 KB LDS, one workgroup per CU): the fused gate/up + SwiGLU once these
// tiles alone cover 3/4 of the CUs (never split: the kernel has no split-K
// path for eight waves).  Llama-1B MLP T = 512 (I x K = 8192 x 2048, graph-free
// timing of 30 calls, cold weights): 48.6 us with 256 x 64 -> 40.6 us; with
// two stages ahead 42.4.  The one-projection shapes measured slower on it
// (they need split K at T = 512)
using CfgS128 = Cfg<4, 2, 2, 2, 2>;

inline size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

struct Plan {
    int tiles_r, tiles_c, nsplit, gps;
};

// No split when the tiles cover 3/4 of the CUs; otherwise split K (whole
// groups, at least min_groups per split) until the grid reaches `target`
// workgroups (the number that can be resident at once).
template <class CF>
Plan make_plan(int R, int C, int G, int cus, int target, int min_groups) {
    Plan pl;
    pl.tiles_r = cdiv(R, CF::BR);
    pl.tiles_c = cdiv(C, CF::BC);
    const int tiles = pl.tiles_r * pl.tiles_c;
    int ns = 4 * tiles >= 3 * cus || CF::NW == 8 ? 1 : target / tiles;
    ns = max(1, min(ns, G / min_groups));
    pl.gps = cdiv(G, ns);
    pl.nsplit = cdiv(G, pl.gps);
    return pl;
}

// `prep(args, extra)` runs before the GEMM with `extra_bytes` of scratch
// (after the split-K partials) and may point args.X / args.xs into it
template <class CF, bool XS, int OUT, class Prep>
clove_status_t run(Args a, int cus, int target, int min_groups, size_t extra_bytes, hipStream_t stream,
                   Prep prep) {
    // OUT 2 (SwiGLU): a tile of BR weight rows makes BR/2 outputs
    const Plan pl = make_plan<CF>(OUT == 2 ? 2 * a.R : a.R, a.C, a.G, cus, target, min_groups);
    a.tiles_r = pl.tiles_r;
    a.tiles_c = pl.tiles_c;
    a.nsplit = pl.nsplit;
    a.gps = pl.gps;
    const int tiles = pl.tiles_r * pl.tiles_c;
    const size_t part_bytes =
        pl.nsplit > 1 ? round256((size_t)tiles * pl.nsplit * CF::NT * CF::FW * CF::FX * 16 * sizeof(float)) : 0;
    char* extra = nullptr;
    if (part_bytes + extra_bytes > 0) {
        Scratch s;
        const clove_status_t st = acquire_scratch(stream, part_bytes + extra_bytes, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        a.part = s.partials;
        a.counters = s.counters;
        extra = reinterpret_cast<char*>(s.partials) + part_bytes;
    }
    const clove_status_t st = prep(a, extra);
    if (st != CLOVE_OK) return st;
    auto k = i4w_gemm<CF, XS, OUT>;
    constexpr int lds = CF::template lds_bytes<XS>();
    static_assert(lds <= 160 * 1024, "LDS");
    if (ensure_lds(reinterpret_cast<const void*>(k), lds) != CLOVE_OK)
        return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, dim3((unsigned)(tiles * pl.nsplit)), dim3(CF::NT), lds, stream, a);
    return check_launch();
}

// Tile choice by the number of X rows C (measured on MI355X):
//   C <= 32: 64 x 32, two waves, three workgroups per CU (HBM-bound)
//   otherwise 128 x 64 with two workgroups per CU, whose waves interleave
//   VALU (unpack, fold) with MFMA -- ahead of 128 x 128 by 15-25 % on the
//   INT4 N = 128 and W4A16 T = 512 shapes -- unless 256 x 128 tiles already
//   cover the CUs (large prefill); the fused SwiGLU from 512 X rows up: 256 x
//   128 with eight waves where those tiles cover 3/4 of the CUs, else 256 x 64
// Splits keep at least 10 (64 x 32) or 8 groups each.
template <bool XS, int OUT, class Prep>
clove_status_t by_shape(const Args& a, int cus, size_t extra_bytes, hipStream_t stream, Prep prep) {
    const int rows = OUT == 2 ? 2 * a.R : a.R;  // weight rows
    if (a.C <= 32) return run<CfgC32, XS, OUT>(a, cus, 3 * cus, 10, extra_bytes, stream, prep);
    if (OUT == 2 && a.C >= 512) {
        if (4 * cdiv(rows, CfgS128::BR) * cdiv(a.C, CfgS128::BC) >= 3 * cus)
            return run<CfgS128, XS, OUT>(a, cus, cus, 8, extra_bytes, stream, prep);
        return run<CfgS64, XS, OUT>(a, cus, 2 * cus, 8, extra_bytes, stream, prep);
    }
    // (SwiGLU tiles pair gate and up rows: the same outputs take twice the
    // weight rows, so the big tile waits for twice the grid)
    if (cdiv(rows, CfgBig::BR) * cdiv(a.C, CfgBig::BC) >= (OUT == 2 ? 2 : 1) * cus)
        return run<CfgBig, XS, OUT>(a, cus, cus, 8, extra_bytes, stream, prep);
    return run<CfgC64, XS, OUT>(a, cus, 2 * cus, 8, extra_bytes, stream, prep);
}

bool fits31(int64_t bytes) { return bytes < ((int64_t)1 << 31); }

// ---- the streaming kernel (i4w_stream.hpp) for C <= 32 X rows ----
template <int WF, int XF, int NG, int KS, bool XS, int OUT, bool RAWB>
clove_status_t launch_stream(const Args& a, hipStream_t stream) {
    using SC = SCfg<WF, XF, NG, KS>;
    const int lds = SC::lds_bytes(a.G, XS, RAWB);
    auto k = i4w_stream<SC, XS, OUT, RAWB>;
    if (ensure_lds(reinterpret_cast<const void*>(k), lds) != CLOVE_OK)
        return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, dim3((unsigned)cdiv(a.R, SC::ROWS)), dim3(SC::NT), lds, stream, a);
    return check_launch();
}

// K slices: the fewest waves (2, 4 or 8) that leave each at most 11 groups,
// unrolled for 8 groups when that suffices
// (BIG_G = false: the caller never passes more than 64 groups, and the
// 11-group, 8-slice variant is not instantiated)
template <int WF, int XF, bool XS, int OUT, bool RAWB = false, bool BIG_G = true>
clove_status_t stream_by_k(const Args& a, hipStream_t stream) {
    const int G = a.G;
    if (G <= 16) return launch_stream<WF, XF, 8, 2, XS, OUT, RAWB>(a, stream);
    if (G <= 22) return launch_stream<WF, XF, 11, 2, XS, OUT, RAWB>(a, stream);
    if (G <= 32) return launch_stream<WF, XF, 8, 4, XS, OUT, RAWB>(a, stream);
    if (G <= 44) return launch_stream<WF, XF, 11, 4, XS, OUT, RAWB>(a, stream);
    if (!BIG_G || G <= 64) return launch_stream<WF, XF, 8, 8, XS, OUT, RAWB>(a, stream);
    if constexpr (BIG_G) return launch_stream<WF, XF, 11, 8, XS, OUT, RAWB>(a, stream);
    return CLOVE_ERR_INVALID_ARG;
}

constexpr int kStreamMaxGroups = 88;  // K <= 11264

// Two weight fragments (32 rows) per workgroup when that still gives every
// CU a workgroup, else one (measured on the 11008 x 4096 and 4096 x 11008
// shapes: 32 rows and 4 slices, 16 rows and 8 slices)
// INT4 (XS) reaches this with at most 16 columns, so only one X fragment.
// Two X fragments with two weight fragments and 11-group slices (K > 8192)
// need more registers than a lane has: those take one weight fragment.
template <bool XS, int OUT>
clove_status_t run_stream(const Args& a, int cus, hipStream_t stream) {
    const bool wf2 = cdiv(a.R, 32) >= cus;
    if (XS || a.C <= 16) return wf2 ? stream_by_k<2, 1, XS, OUT>(a, stream) : stream_by_k<1, 1, XS, OUT>(a, stream);
    if constexpr (!XS) {
        if (wf2 && a.G <= 64) return stream_by_k<2, 2, XS, OUT, false, false>(a, stream);
        return stream_by_k<1, 2, XS, OUT>(a, stream);
    }
    return CLOVE_ERR_INVALID_ARG;
}

// Every workgroup of the streaming kernel reads all of X (C rows x K fp16),
// so its cost grows with C x K per CU, while the split-K MFMA kernel reads
// each X tile once per 64 weight rows and is flat in C.  Measured (W4A16,
// T = 5..32 on 8192x2048, 2048x8192, 4096x4096, 4096x11008, 11008x4096): the
// stream is ahead below ~256 KB of X per CU, counting one copy per round of
// workgroups on a CU, and the MFMA kernel from there (4096x11008 T = 32:
// 26.3 against 16.4 us; 2048x8192 T = 16: 12.2 against 10.8 us).
bool stream_ahead(const Args& a, int cus) {
    const bool wf2 = cdiv(a.R, 32) >= cus && (a.C <= 16 || a.G <= 64);  // run_stream's weight fragments
    const int64_t rounds = cdiv(cdiv(a.R, wf2 ? 32 : 16), cus);
    return (int64_t)a.C * a.K * 2 * rounds < 256 * 1024;
}

}  // namespace

bool try_i4w_w4a16(const W4A16Args& w, int cus, hipStream_t stream, clove_status_t* status) {
    // three or four tokens on large weights: the streaming kernel rather than
    // the GEMV (cold, T = 4: 4096x11008 12.1 against 22.0 us, 4096x4096 5.8
    // against 8.0; 2048x2048 stays on the GEMV, 4.2 against 4.6)
    const bool small_t = w.T <= 2 || (w.T <= 4 && (int64_t)w.O * w.K <= ((int64_t)8 << 20));
    if (small_t || w.K <= 0 || w.K % 128 != 0 || !aligned16(w.X) || !aligned16(w.W)) return false;
    if (!fits31((int64_t)w.T * w.K * 2) || !fits31((int64_t)w.O * (w.K / 2))) return false;
    Args a{};
    a.W = w.W;
    a.wscale = w.scale;
    a.wzero = w.zero;
    a.X = w.X;
    a.out = w.Y;
    a.R = w.O;
    a.C = w.T;
    a.K = w.K;
    a.G = w.K / 128;
    a.alpha = w.alpha;
    a.beta = w.beta;
    if (w.T <= 32 && a.G <= kStreamMaxGroups && stream_ahead(a, cus)) {
        *status = run_stream<false, 1>(a, cus, stream);
        return true;
    }
    if (w.T <= 4) return false;  // (the GEMV, outside the stream's domain)
    *status = by_shape<false, 1>(a, cus, 0, stream, [](Args&, char*) { return CLOVE_OK; });
    return true;
}

bool try_i4w_w4a16_swiglu(const W4A16Args& w, int cus, hipStream_t stream, clove_status_t* status) {
    if (w.T <= 4 || w.K <= 0 || w.K % 128 != 0 || !aligned16(w.X) || !aligned16(w.W)) return false;
    if (!fits31((int64_t)w.T * w.K * 2) || !fits31((int64_t)2 * w.O * (w.K / 2))) return false;
    Args a{};
    a.W = w.W;
    a.wscale = w.scale;
    a.wzero = w.zero;
    a.X = w.X;
    a.out = w.Y;
    a.R = w.O;  // outputs; the weight has 2 O rows (gate, then up)
    a.C = w.T;
    a.K = w.K;
    a.G = w.K / 128;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    *status = by_shape<false, 2>(a, cus, 0, stream, [](Args&, char*) { return CLOVE_OK; });
    return true;
}

bool try_i4w_int4_rawb(const Int4Args& q, int cus, hipStream_t stream, clove_status_t* status);

bool try_i4w_int4(const Int4Args& q, int cus, hipStream_t stream, clove_status_t* status) {
    if (try_i4w_int4_rawb(q, cus, stream, status)) return true;
    if (q.mode != CLOVE_INT4_GROUPWISE || q.N <= 8 || q.K <= 0 || q.K % 128 != 0 || !aligned16(q.A))
        return false;
    const int Npad = (q.N + 63) / 64 * 64;
    const int G = q.K / 128;
    if (!fits31((int64_t)Npad * q.K * 2) || !fits31((int64_t)q.M * (q.K / 2))) return false;
    const size_t xt_bytes = round256((size_t)Npad * q.K * 2);
    const size_t xs_bytes = round256((size_t)G * Npad * 4);
    Args a{};
    a.W = q.A;
    a.wscale = q.A_scale;
    a.wzero = q.A_zero;
    a.out = q.C;
    a.R = q.M;
    a.C = q.N;
    a.K = q.K;
    a.G = G;
    a.ldxs = Npad;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    const int ldb = (q.N + 1) / 2;
    auto prep = [&](Args& args, char* extra) -> clove_status_t {
        uint16_t* xt = reinterpret_cast<uint16_t*>(extra);
        float* xs = reinterpret_cast<float*>(extra + xt_bytes);
        CLOVE_LAUNCH(i4w_prep_b, dim3((unsigned)G, (unsigned)cdiv(Npad, 128)), dim3(256), 0, stream, q.B,
                           ldb, q.B_scale, q.B_zero, q.N, q.K, G, Npad, xt, xs);
        args.X = xt;
        args.xs = xs;
        return check_launch();
    };
    if (q.N <= 16 && G <= kStreamMaxGroups) {
        // the B transpose into scratch, then the streaming kernel
        Scratch s;
        clove_status_t st = acquire_scratch(stream, xt_bytes + xs_bytes, 0, &s);
        if (st == CLOVE_OK) st = prep(a, reinterpret_cast<char*>(s.partials));
        if (st == CLOVE_OK) st = run_stream<true, 0>(a, cus, stream);
        *status = st;
        return true;
    }
    *status = by_shape<true, 0>(a, cus, xt_bytes + xs_bytes, stream, prep);
    return true;
}

// Weight rows per workgroup of the raw-B stream, 16 WF (WF = 1..3): the fewest
// rows on the busiest CU, counting whole rounds of workgroups; on a tie the
// larger workgroups when each has four or more K-slice waves (G > 16), else
// the smaller.  Cold graph replays, us per call for WF = 1 / 2 / 3 (N = 16):
// 11008 x 4096 9.57 / 11.23 / 9.09, 11008 x 8192 19.73 / 20.62 / 15.90,
// 8192 x 4096 7.58 / 7.30 / 8.66, 16384 x 4096 12.06 / 11.17 / 14.40,
// 4096 x 4096 5.52 / 6.87 / 8.29, 14336 x 2048 7.48 / 9.15 / 11.13, 11008 x
// 2048 7.17 / 8.98 / 7.81: the rule picks the fastest of the three in each.
int rawb_wf(int R, int G, int cus) {
    int best = 1;
    int64_t best_rows = -1;
    for (int wf = 1; wf <= 3; ++wf) {
        const int64_t rows = (int64_t)cdiv(cdiv(R, 16 * wf), cus) * wf;
        if (best_rows < 0 || rows < best_rows || (rows == best_rows && G > 16)) {
            best = wf;
            best_rows = rows;
        }
    }
    return best;
}

bool try_i4w_int4_rawb(const Int4Args& q, int cus, hipStream_t stream, clove_status_t* status) {
    // 15 or 16 columns: B rows are 8 bytes, read in place (no transpose pass)
    const int G = q.K / 128;
    if (q.mode != CLOVE_INT4_GROUPWISE || (q.N != 15 && q.N != 16) || q.K <= 0 || q.K % 128 != 0 ||
        G > kStreamMaxGroups || !aligned16(q.A) || !aligned16(q.B) || !fits31((int64_t)q.M * (q.K / 2)))
        return false;
    Args a{};
    a.W = q.A;
    a.wscale = q.A_scale;
    a.wzero = q.A_zero;
    a.out = q.C;
    a.R = q.M;
    a.C = q.N;
    a.K = q.K;
    a.G = G;
    a.B = q.B;
    a.bscale = q.B_scale;
    a.bzero = q.B_zero;
    a.N = q.N;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    const int wf = rawb_wf(a.R, G, cus);
    *status = wf == 3   ? stream_by_k<3, 1, true, 0, true>(a, stream)
              : wf == 2 ? stream_by_k<2, 1, true, 0, true>(a, stream)
                        : stream_by_k<1, 1, true, 0, true>(a, stream);
    return true;
}

}  // namespace clove
