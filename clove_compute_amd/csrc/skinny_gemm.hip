// Host side of the skinny GEMM (skinny_gemm.hpp): tile configuration by M,
// split-K plan, scratch.
#include "dispatch.hpp"
#include "skinny_gemm.hpp"

namespace clove {
namespace {

using namespace sk;

// (I8, BM, BN, WM, WN, stages)
using F16M32 = Cfg<false, 32, 128, 1, 4, 5>;
using F16M128 = Cfg<false, 128, 64, 4, 1, 4>;
// mid-size shapes (M > 256) whose 256x256 tile grid would leave CUs idle:
// 128x128 tiles (waves of 64x64), or 64x64 tiles when even those are too few
// (hot launches: 2048^3 25 us with 128x128 against 45 us on the generic
// register-staged kernel; 1024^3 8 us with 64x64 against 13 us with 128x128
// and 21 us generic; 512x4096x4096 29 us with 128x128 in two K splits
// against 33 us with 128x64)
using F16T128 = Cfg<false, 128, 128, 2, 2, 3>;
using F16T64 = Cfg<false, 64, 64, 2, 2, 6>;
// the same tile one stage ahead for K <= 512: every workgroup's first stage
// then waits behind a smaller burst of the whole grid's prologue loads (512^3:
// 5.5 -> 4.7 us; from K = 1024 the six stages are ahead, 1024^3 8.7 against
// 13.2 us)
using F16T64S2 = Cfg<false, 64, 64, 2, 2, 2>;
// small products (short K, at most one 32x32 tile per CU): 32x32 tiles whose
// four waves take one k-step of every K tile each, two stages ahead -- 4x the
// workgroups of 64x64 tiles at a quarter of the operand bytes each (hot graph
// replays, us per call, against the 64x64 / 32x128 tiles: 512^3 4.98 / 5.61
// -> 4.27, 512 x 512 x 1024 6.90 / 7.83 -> 5.51, 64 x 4096 x 1024 6.91 / 7.83
// -> 5.49, 3 x 8192 x 1024 6.72 / 7.71 -> 5.33, 100 x 200 x 320 4.04 / 4.53
// -> 3.67; one or three stages ahead no faster; at 512 such tiles and more it
// only ties or loses: 512 x 1024 x 512 5.27 -> 5.21, 1024 x 1024 x 512 5.81
// -> 7.13)
using F16K32 = Cfg<false, 32, 32, 1, 1, 3, 1, 4>;
using I8M32 = Cfg<true, 32, 128, 1, 4, 5>;
using I8M128 = Cfg<true, 128, 64, 4, 1, 4>;
using I8T128 = Cfg<true, 128, 128, 2, 2, 3>;

template <class CF, int OUT>
clove_status_t run(Args a, int batch, int cus, hipStream_t stream) {
    a.tiles_m = cdiv(a.M, CF::BM);
    a.tiles_n = cdiv(a.N, CF::BN);
    a.batch = batch;
    const int tiles = a.tiles_m * a.tiles_n * batch;
    const int nk = a.K / CF::BK;
    // split K (whole K tiles, at least two per split) until about one
    // workgroup per CU; not for short K (<= 16 K tiles), where the split's
    // publish / count / reload tail costs more than the shorter stream saves
    // (512^3: 8.4 us with 4 splits, 7.2 us with none, measured)
    int ns = tiles >= cus ? 1 : cus / tiles;
    ns = max(1, min(ns, nk / 2));
    if (nk <= 16 || CF::KW > 1) ns = 1;
    const int kt_per = cdiv(nk, ns);
    a.kps = kt_per * CF::BK;
    a.nsplit = cdiv(nk, kt_per);
    if (a.nsplit > 1) {
        Scratch s;
        const size_t bytes = (size_t)tiles * a.nsplit * CF::NT * CF::NB * CF::FM * CF::FN * 16 * sizeof(float);
        const clove_status_t st = acquire_scratch(stream, bytes, (size_t)tiles, &s);
        if (st != CLOVE_OK) return st;
        a.part = s.partials;
        a.counters = s.counters;
    }
    auto k = skinny_gemm<CF, OUT>;
    if (ensure_lds(reinterpret_cast<const void*>(k), CF::LDS) != CLOVE_OK)
        return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, dim3((unsigned)(tiles * a.nsplit)), dim3(CF::NT), CF::LDS, stream, a);
    return check_launch();
}

bool fits31(int64_t bytes) { return bytes < ((int64_t)1 << 31); }

// The FP16 tile shapes, chosen by shape alone (so that the fused SwiGLU below
// picks the same tiles, and with them the same split plan, as the two GEMMs
// it replaces).
enum class F16Tile { kM32, kM128, kT128, kT64, kK32 };

F16Tile pick_f16_tile(int batch, int M, int N, int K, int cus) {
    const bool short_k = K <= 16 * F16M128::BK;  // no split K (see run)
    const bool long_k = K >= 4096;
    if (short_k && (int64_t)cdiv(M, F16K32::BM) * cdiv(N, F16K32::BN) * batch <= cus) return F16Tile::kK32;
    // 128x128 tiles, split K when they are few: for M > 256 once they cover
    // half the CUs or K is long, for 128 < M <= 256 on long K and N >= 4096
    // (cold weights, against 64x64 tiles for M > 256 and 128x64 up to 256:
    // 11008x4096 at M = 192 44.3 against 64.2 us, 4096x11008 at M = 384 64.1
    // against 108.6 us, 4096x4096 at M = 384 30.6 against 43.7 us, 2048x8192
    // at M = 512 35.2 against 47.4 us; K = 2048 and N = 2048 stay as they
    // were: 2048x2048 at M = 384 14.0 with 64x64 against 19.0, 2048x8192 at
    // M = 160 24.0 with 128x64 against 26.0; 64x64 for short K with few tiles:
    // 1024^3 8 us against 13)
    if (M > 256) {
        const int64_t t128 = (int64_t)cdiv(M, 128) * cdiv(N, 128) * batch;
        return (t128 >= cus / 2 || long_k) ? F16Tile::kT128 : F16Tile::kT64;
    }
    if (M > 128 && long_k && N >= 4096) return F16Tile::kT128;
    // and for 64 < M <= 128 on wide weights (N >= 10240, K >= 4096), in two K
    // splits: half the A-panel bytes per workgroup of the 128x64 tiles (cold,
    // 128 x 11008 x 4096 35.1 -> 30.2 us, 96 x 11008 x 4096 31.2 -> 28.5,
    // 80 x 11008 x 4096 30.8 -> 27.7, 128 x 14336 x 4096 39.0 -> 34.1; not at
    // N = 8192, K = 2048 or N = 4096, K = 11008, where 128x64 stays ahead)
    if (M > 64 && M <= 128 && long_k && N >= 10240) return F16Tile::kT128;
    // 32-row tiles up to M = 64 (cold 4096 x 4096 weights: M = 40 / 48 / 64 at
    // 13.6 / 14.1 / 14.5 us against 14.9 / 15.3 / 15.5 with 64-row tiles), and
    // for short K with few 128-row tiles, where they make 4x the workgroups
    // without a split (512^3: 6.1 us against 7.2, measured)
    const bool few = (int64_t)cdiv(M, F16M128::BM) * cdiv(N, F16M128::BN) * batch < cus / 2;
    if (M <= 64 || (short_k && few)) return F16Tile::kM32;
    return F16Tile::kM128;
}

bool f16_domain(const void* A, const void* B, const void* C, int M, int N, int K) {
    if (M <= 1 || K <= 0 || K % 64 != 0 || N < 8 || N % 8 != 0) return false;
    if (M <= 4 && !skinny_before_gemv(M, N, K)) return false;
    if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return false;
    // (the DMA offsets of the padded rows m < M + 128 must stay 32-bit)
    return fits31((int64_t)(M + 128) * K * 2) && fits31((int64_t)K * N * 2) && fits31((int64_t)M * N * 2);
}

// two-B-operand (gate, up) counterparts of the tiles above; fewer stages
// where both B tiles would not fit the LDS
using SwM32 = Cfg<false, 32, 128, 1, 4, 4, 2>;
using SwM128 = Cfg<false, 128, 64, 4, 1, 4, 2>;
using SwT128 = Cfg<false, 128, 128, 2, 2, 3, 2>;
using SwT64 = Cfg<false, 64, 64, 2, 2, 6, 2>;
using SwK32 = Cfg<false, 32, 32, 1, 1, 3, 2, 4>;

}  // namespace

bool try_skinny_fp16(const uint16_t* A, const uint16_t* B, uint16_t* C, int batch, int M, int N, int K,
                     float alpha, float beta, int cus, hipStream_t stream, clove_status_t* status) {
    if (!f16_domain(A, B, C, M, N, K)) return false;
    Args a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.alpha = alpha;
    a.beta = beta;
    a.M = M;
    a.N = N;
    a.K = K;
    a.sA = (int64_t)M * K;
    a.sB = (int64_t)K * N;
    a.sC = (int64_t)M * N;
    switch (pick_f16_tile(batch, M, N, K, cus)) {
        case F16Tile::kM32: *status = run<F16M32, kF16AlphaBeta>(a, batch, cus, stream); break;
        case F16Tile::kM128: *status = run<F16M128, kF16AlphaBeta>(a, batch, cus, stream); break;
        case F16Tile::kT128: *status = run<F16T128, kF16AlphaBeta>(a, batch, cus, stream); break;
        case F16Tile::kT64:
            *status = K <= 512 ? run<F16T64S2, kF16AlphaBeta>(a, batch, cus, stream)
                               : run<F16T64, kF16AlphaBeta>(a, batch, cus, stream);
            break;
        case F16Tile::kK32: *status = run<F16K32, kF16AlphaBeta>(a, batch, cus, stream); break;
    }
    return true;
}

bool try_skinny_swiglu(const uint16_t* X, const uint16_t* W_gate, const uint16_t* W_up, uint16_t* out, int T,
                       int hidden, int inter, int cus, hipStream_t stream, clove_status_t* status) {
    if (!f16_domain(X, W_gate, out, T, inter, hidden) || !aligned16(W_up)) return false;
    Args a{};
    a.A = X;
    a.B = W_gate;
    a.B2 = W_up;
    a.C = out;
    a.alpha = 1.0f;
    a.M = T;
    a.N = inter;
    a.K = hidden;
    a.sA = (int64_t)T * hidden;
    a.sB = (int64_t)hidden * inter;
    a.sC = (int64_t)T * inter;
    switch (pick_f16_tile(1, T, inter, hidden, cus)) {
        case F16Tile::kM32: *status = run<SwM32, kF16SwiGLU>(a, 1, cus, stream); break;
        case F16Tile::kM128: *status = run<SwM128, kF16SwiGLU>(a, 1, cus, stream); break;
        case F16Tile::kT128: *status = run<SwT128, kF16SwiGLU>(a, 1, cus, stream); break;
        case F16Tile::kT64: *status = run<SwT64, kF16SwiGLU>(a, 1, cus, stream); break;
        case F16Tile::kK32: *status = run<SwK32, kF16SwiGLU>(a, 1, cus, stream); break;
    }
    return true;
}

bool try_skinny_int8(const Int8Args& q, int cus, hipStream_t stream, clove_status_t* status) {
    if (q.M <= 2 || q.M > 2048 || q.K <= 0 || q.K % 128 != 0 || q.N < 16 || q.N % 16 != 0) return false;
    // three or four rows: the GEMV unless the weight is large (cold 11008 x 4096
    // and 4096 x 11008, M = 3 / 4: 13.9 / 17.1 us here against 21.7 / 20.5 us
    // on the GEMV; at 4096 x 4096 the GEMV is ahead, 9.2 against 11.5 us)
    if (q.M <= 4 && (int64_t)q.N * q.K <= ((int64_t)32 << 20)) return false;
    if (q.za != 0 || q.zb != 0 || !aligned16(q.A) || !aligned16(q.B) || !aligned16(q.C)) return false;
    if (!fits31((int64_t)(q.M + 128) * q.K) || !fits31((int64_t)q.K * q.N) || !fits31((int64_t)q.M * q.N * 4))
        return false;
    Args a{};
    a.A = q.A;
    a.B = q.B;
    a.C = q.C;
    a.sa = q.sa;
    a.sb = q.sb;
    a.scale = q.scale;
    a.M = q.M;
    a.N = q.N;
    a.K = q.K;
    auto pick = [&](auto out_tag) -> clove_status_t {
        constexpr int OUT = decltype(out_tag)::value;
        // 32-row tiles up to M = 64, and up to 128 unless the weight is large
        // (cold: 4096 x 4096 at M = 64 / 128 10.8 / 13.8 us against 15.0 / 15.3
        // with 64- and 128-row tiles, 8192 x 2048 at M = 128 12.0 against 14.7;
        // 11008 x 4096 at M = 128 24.2 with 128-row tiles against 30.6), from
        // M = 160 the 128-row tiles, and for short K as for FP16.  Up to
        // M = 2048 this kernel is ahead of the register-staged MFMA GEMM
        // (4096 x 4096 at M = 768 / 2048 43.4 / 79.4 us against 66.8 / 156.1,
        // 11008 x 4096 at M = 768 95.3 against 209.2); at M = 4096 it is not.
        const bool short_k = q.K <= 16 * I8M128::BK &&
                             (int64_t)cdiv(q.M, I8M128::BM) * cdiv(q.N, I8M128::BN) < cus / 2;
        const bool large_w = (int64_t)q.N * q.K > ((int64_t)32 << 20);
        if (q.M <= 64 || (q.M <= 128 && !large_w) || short_k) return run<I8M32, OUT>(a, 1, cus, stream);
        // 128x128 tiles for M <= 128 on wide weights, as for FP16 (cold, 128 x
        // 11008 x 4096 23.7 -> 20.5 us; 128 x 4096 x 11008 stays on 128x64)
        if (q.M <= 128 && q.N >= 10240 && q.K >= 4096) return run<I8T128, OUT>(a, 1, cus, stream);
        return run<I8M128, OUT>(a, 1, cus, stream);
    };
    switch (q.out) {
        case Int8Out::kHalfPerTensor: *status = pick(std::integral_constant<int, kI8Tensor>{}); break;
        case Int8Out::kHalfRowCol: *status = pick(std::integral_constant<int, kI8RowCol>{}); break;
        case Int8Out::kAcc32: *status = pick(std::integral_constant<int, kI8Acc32>{}); break;
        default: return false;
    }
    return true;
}

}  // namespace clove
