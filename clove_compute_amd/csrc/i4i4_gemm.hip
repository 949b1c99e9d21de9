// Host side of the group-wise INT4 x INT4 int8-MFMA GEMM (i4i4_gemm.hpp):
// eligibility, the Bt pre-pass, tile / split-K plan and scratch.
#include "dispatch.hpp"
#include "i4i4_gemm.hpp"

namespace clove {
namespace {

using namespace i4i4;

bool fits31(int64_t bytes) { return bytes < ((int64_t)1 << 31); }
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// One workgroup per CU (the rings take most of the LDS): 64-row tiles, split
// over groups until the grid reaches the CUs, never past them (a second round
// of workgroups would double the time), at least two groups per split.
struct Plan {
    int tiles_m, nsplit, gps;
};

Plan plan_for(int M, int tiles_n, int G, int cus) {
    Plan pl{};
    pl.tiles_m = cdiv(M, BR);
    const int tiles = pl.tiles_m * tiles_n;
    int ns = tiles >= cus ? 1 : cus / tiles;
    ns = max(1, min(ns, G / 2));
    // (an even number of groups per split: every stage starts on an even group,
    // whose (g, g + 1) pair of zA / sA is one aligned dword)
    pl.gps = 2 * cdiv(cdiv(G, ns), 2);
    pl.nsplit = cdiv(G, pl.gps);
    return pl;
}

}  // namespace

namespace {

// The shared body of the GEMM and the partials hook: plan, scratch, the Bt
// pre-pass, the launch.  P != null selects the partials mode (scales unused).
clove_status_t run(const Int4Args& q, int32_t* P, int cus, hipStream_t stream) {
    const int G = q.K / 128;
    const int Npad = cdiv(q.N, BC) * BC;
    Args a{};
    a.A = q.A;
    // (the partials mode never reads the scales; its weight DMA still needs a
    // valid [M, G] fp16 array to read from)
    a.sA = P ? q.A_zero : q.A_scale;
    a.zA = q.A_zero;
    a.C = q.C;
    a.P = P;
    a.M = q.M;
    a.N = q.N;
    a.K = q.K;
    a.G = G;
    a.Npad = Npad;
    a.tiles_n = Npad / BC;
    const Plan pl = plan_for(q.M, a.tiles_n, G, cus);
    a.tiles_m = pl.tiles_m;
    a.nsplit = pl.nsplit;
    a.gps = pl.gps;
    a.vec_store = (q.N % 8 == 0) && aligned16(q.C);
    const int tiles = a.tiles_m * a.tiles_n;
    const size_t slab = (size_t)BR * BC * 4;  // one fp32 partial tile
    const size_t part_bytes = !P && a.nsplit > 1 ? (size_t)tiles * a.nsplit * slab : 0;
    const size_t bt_bytes = round256((size_t)Npad * q.K);
    const size_t sb_bytes = round256((size_t)G * Npad * 4);
    Scratch s;
    clove_status_t st = acquire_scratch(stream, part_bytes + bt_bytes + sb_bytes, (size_t)tiles, &s);
    if (st != CLOVE_OK) return st;
    char* base = reinterpret_cast<char*>(s.partials);
    a.part = s.partials;
    a.counters = s.counters;
    int8_t* bt = reinterpret_cast<int8_t*>(base + part_bytes);
    float* sbf = reinterpret_cast<float*>(base + part_bytes + bt_bytes);
    a.Bt = bt;
    a.sBf = sbf;
    const int ldb = (q.N + 1) / 2;
    CLOVE_LAUNCH(i4_prep_bt, dim3((unsigned)G, (unsigned)(Npad / PREP_COLS)), dim3(128), 0, stream, q.B, ldb,
                 P ? nullptr : q.B_scale, q.B_zero, q.N, q.K, Npad, bt, sbf);
    auto k = P ? i4i4_gemm<true> : i4i4_gemm<false>;
    if (ensure_lds(reinterpret_cast<const void*>(k), LDS) != CLOVE_OK)
        return CLOVE_ERR_LAUNCH;
    CLOVE_LAUNCH(k, dim3((unsigned)(tiles * a.nsplit)), dim3(NT), LDS, stream, a);
    return check_launch();
}

// K a multiple of 256 (whole two-group stages; every (g, g + 1) fp16 pair of
// zA / sA is one aligned dword), a 16-byte aligned A, and offsets that fit
// the 32-bit buffer ranges
bool eligible(const Int4Args& q) {
    if (q.K <= 0 || q.K % 256 != 0 || !aligned16(q.A)) return false;
    const int G = q.K / 128;
    const int Npad = cdiv(q.N, BC) * BC;
    return fits31((int64_t)(q.M + BR) * (q.K / 2)) && fits31((int64_t)Npad * q.K) &&
           fits31((int64_t)q.M * G * 2) && fits31((int64_t)G * Npad * 4);
}

}  // namespace

// Group-wise mode with N >= 64 columns (fewer go to the GEMV / streaming
// kernels).
bool try_i4i4(const Int4Args& q, int cus, hipStream_t stream, clove_status_t* status) {
    if (q.mode != CLOVE_INT4_GROUPWISE || q.N < 64 || !eligible(q)) return false;
    *status = run(q, nullptr, cus, stream);
    return true;
}

clove_status_t launch_i4i4_partials(const Int4Args& q, int32_t* P, int cus, hipStream_t stream) {
    if (!eligible(q)) return CLOVE_ERR_INVALID_ARG;
    return run(q, P, cus, stream);
}

}  // namespace clove
