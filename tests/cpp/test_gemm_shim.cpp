// Drop-in check of the C++ shim include/clove/gemm.h, written the way the
// reference's own C++ callers use its API (namespace clove, same names,
// argument order and defaults; cudaStream_t -> hipStream_t):
//
//  * the six GEMM cases of the reference's test program (tests/test_gemm.cu:
//    small 64^3 :99-121, medium 256^3 :123-145, large 1024^3 :147-169,
//    nonsquare 128x4096x4096 :171-194, decode 1x4096x4096 :196-219,
//    alpha/beta :221-243, which the reference only smoke-runs; here it is
//    checked), each judged by the reference's comparison rule (an element
//    fails iff rel > 0.05 and abs > 1e-3, rel = |a - b| / (|b| + 1e-3),
//    tests/test_gemm.cu:22-58) and by the tighter rule of this repository's
//    tests (|a - b| <= 1e-2 max(|b|, 1e-2 rms(b))), against the float64 oracle;
//  * gemm_int8 (bit-exact), gemm_int4 group-wise (tolerance) and through
//    gemm_int4_ex the reference-literal mode (bit-exact), gemm_fp16_batched,
//    swiglu and gemm_w4a16 / w4a16_swiglu, the calls of the runtime's layer
//    (src/runtime/inference.cu:139-194) on INT4 weights.
//
// Built by __graft_entry__.build() next to this file; run by
// tests/test_cpp_shim.py on the GPU.  Exit status 0 iff every case passes.
#include <clove/gemm.h>

#include "../../oracle/clove_oracle.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

struct Rng {  // splitmix64
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    float uniform(float lo, float hi) { return lo + (hi - lo) * (float)((next() >> 40) * (1.0 / 16777216.0)); }
    int integer(int lo, int hi) { return lo + (int)(next() % (uint64_t)(hi - lo + 1)); }  // [lo, hi]
};

std::vector<uint16_t> rand_f16(size_t n, float lo, float hi, Rng& g) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = oracle_f32_to_f16(g.uniform(lo, hi));
    return v;
}

// element type of a host vector, as the reference's Tensor records it
// (src/runtime/tensor.cu:62-65 sizes a buffer as numel * dtype_size(dtype))
template <class T> constexpr clove::DType dtype_of();
template <> constexpr clove::DType dtype_of<uint16_t>() { return clove::DType::FP16; }
template <> constexpr clove::DType dtype_of<int8_t>() { return clove::DType::INT8; }
template <> constexpr clove::DType dtype_of<uint8_t>() { return clove::DType::INT8; }  // packed INT4 bytes

// the reference's error convention around every runtime call
// (include/clove/common.cuh:11-27)
template <class T>
T* to_dev(const std::vector<T>& h) {
    static_assert(sizeof(T) == 1 || sizeof(T) == 2, "element size");
    const size_t bytes = h.size() * clove::dtype_size(dtype_of<T>());
    T* d = nullptr;
    CLOVE_CHECK_CUDA(hipMalloc(&d, bytes + 16));
    CLOVE_CHECK_CUDA(hipMemcpy(d, h.data(), bytes, hipMemcpyHostToDevice));
    return d;
}

template <class T>
std::vector<T> to_host(const T* d, size_t n) {
    std::vector<T> h(n);
    CLOVE_SYNC_CHECK();
    CLOVE_CHECK_CUDA(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

half* H(uint16_t* p) { return reinterpret_cast<half*>(p); }

int g_failed = 0;

// both rules against the float64 reference
bool compare(const char* name, const std::vector<uint16_t>& got, const std::vector<double>& ref) {
    double rms = 0.0;
    for (double r : ref) rms += r * r;
    rms = std::sqrt(rms / (double)ref.size());
    size_t ref_rule_fail = 0, tol_fail = 0;
    double max_rel = 0.0;
    for (size_t i = 0; i < ref.size(); ++i) {
        const double a = oracle_f16_to_f32(got[i]), b = ref[i];
        const double abs_err = std::fabs(a - b), rel = abs_err / (std::fabs(b) + 1e-3);
        if (!std::isfinite(a) || (rel > 0.05 && abs_err > 1e-3)) ++ref_rule_fail;
        if (!std::isfinite(a) || abs_err > 1e-2 * std::fmax(std::fabs(b), 1e-2 * rms)) ++tol_fail;
        max_rel = std::fmax(max_rel, rel);
    }
    const bool ok = ref_rule_fail == 0 && tol_fail == 0;
    std::printf("%-34s %s  (reference rule: %zu of %zu fail; tolerance: %zu fail; max rel %.2e)\n", name,
                ok ? "PASS" : "FAIL", ref_rule_fail, ref.size(), tol_fail, max_rel);
    if (!ok) ++g_failed;
    return ok;
}

bool compare_bits(const char* name, const std::vector<uint16_t>& got, const std::vector<uint16_t>& ref) {
    size_t bad = 0;
    for (size_t i = 0; i < ref.size(); ++i) bad += got[i] != ref[i];
    std::printf("%-34s %s  (%zu of %zu elements differ)\n", name, bad ? "FAIL" : "PASS", bad, ref.size());
    if (bad) ++g_failed;
    return bad == 0;
}

// ---- the reference's FP16 cases ----
void fp16_case(const char* name, int M, int N, int K, float alpha, float beta, uint64_t seed) {
    Rng g(seed);
    auto A = rand_f16((size_t)M * K, -1.0f, 1.0f, g);
    auto B = rand_f16((size_t)K * N, -1.0f, 1.0f, g);
    auto C0 = rand_f16((size_t)M * N, -1.0f, 1.0f, g);
    uint16_t *dA = to_dev(A), *dB = to_dev(B), *dC = to_dev(C0);
    clove::gemm_fp16(H(dA), H(dB), H(dC), M, N, K, alpha, beta);  // defaults: stream 0
    CLOVE_CHECK_LAST();  // as the reference's launcher does after its kernel (gemm_fp16.cu:304)
    auto got = to_host(dC, (size_t)M * N);
    std::vector<double> ref((size_t)M * N);
    oracle_gemm_fp16_f64(A.data(), B.data(), beta != 0.0f ? C0.data() : nullptr, ref.data(), M, N, K, alpha, beta);
    compare(name, got, ref);
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(dC);
}

void fp16_default_args_case() {
    // the call with the default alpha, beta and stream (src/main.cpp:76, tests/test_gemm.cu)
    const int M = 256, N = 256, K = 256;
    Rng g(11);
    auto A = rand_f16((size_t)M * K, -1.0f, 1.0f, g);
    auto B = rand_f16((size_t)K * N, -1.0f, 1.0f, g);
    std::vector<uint16_t> C0((size_t)M * N, 0x7e00);  // NaN: beta = 0 must not read C
    uint16_t *dA = to_dev(A), *dB = to_dev(B), *dC = to_dev(C0);
    clove::gemm_fp16(H(dA), H(dB), H(dC), M, N, K);
    auto got = to_host(dC, (size_t)M * N);
    std::vector<double> ref((size_t)M * N);
    oracle_gemm_fp16_f64(A.data(), B.data(), nullptr, ref.data(), M, N, K, 1.0, 0.0);
    compare("gemm_fp16 default args 256^3", got, ref);
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(dC);
}

void batched_case() {
    const int batch = 3, M = 96, N = 80, K = 72;
    Rng g(21);
    auto A = rand_f16((size_t)batch * M * K, -1.0f, 1.0f, g);
    auto B = rand_f16((size_t)batch * K * N, -1.0f, 1.0f, g);
    auto C0 = rand_f16((size_t)batch * M * N, -1.0f, 1.0f, g);
    uint16_t *dA = to_dev(A), *dB = to_dev(B), *dC = to_dev(C0);
    clove::gemm_fp16_batched(H(dA), H(dB), H(dC), batch, M, N, K, 0.5f, 1.0f);
    auto got = to_host(dC, (size_t)batch * M * N);
    std::vector<double> ref((size_t)batch * M * N);
    for (int b = 0; b < batch; ++b)
        oracle_gemm_fp16_f64(A.data() + (size_t)b * M * K, B.data() + (size_t)b * K * N, C0.data() + (size_t)b * M * N,
                             ref.data() + (size_t)b * M * N, M, N, K, 0.5, 1.0);
    compare("gemm_fp16_batched 3x96x80x72", got, ref);
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(dC);
}

// ---- INT8, per-tensor scale and zero point: bit-exact ----
void int8_case(int M, int N, int K) {
    Rng g(31 + M);
    std::vector<int8_t> A((size_t)M * K), B((size_t)K * N);
    for (auto& x : A) x = (int8_t)g.integer(-127, 127);
    for (auto& x : B) x = (int8_t)g.integer(-127, 127);
    const float sa = 0.0123f, sb = 0.0071f;
    const int8_t za = 3, zb = -5;
    int8_t *dA = to_dev(A), *dB = to_dev(B);
    uint16_t* dC = to_dev(std::vector<uint16_t>((size_t)M * N, 0));
    clove::gemm_int8(dA, dB, H(dC), M, N, K, sa, za, sb, zb);
    auto got = to_host(dC, (size_t)M * N);
    std::vector<uint16_t> ref((size_t)M * N);
    oracle_gemm_int8(A.data(), B.data(), ref.data(), nullptr, M, N, K, sa, za, sb, zb);
    char name[64];
    std::snprintf(name, sizeof name, "gemm_int8 %dx%dx%d", M, N, K);
    compare_bits(name, got, ref);
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(dC);
}

// ---- INT4: group-wise (tolerance) and the reference-literal mode (bit-exact) ----
void int4_case(int M, int N, int K) {
    Rng g(41 + N);
    const int G = clove::cdiv(K, clove::INT4_GROUP_SIZE), ldb = clove::cdiv(N, 2);
    std::vector<uint8_t> A((size_t)M * (K / 2)), B((size_t)K * ldb);
    for (auto& x : A) x = (uint8_t)g.integer(0, 255);
    for (auto& x : B) x = (uint8_t)g.integer(0, 255);
    auto sA = rand_f16((size_t)M * G, 0.001f, 0.02f, g), sB = rand_f16((size_t)G * N, 0.001f, 0.02f, g);
    std::vector<uint16_t> zA((size_t)M * G), zB((size_t)G * N);
    for (auto& x : zA) x = oracle_f32_to_f16((float)g.integer(0, 15));
    for (auto& x : zB) x = oracle_f32_to_f16((float)g.integer(0, 15));
    uint8_t *dA = to_dev(A), *dB = to_dev(B);
    uint16_t *dsA = to_dev(sA), *dsB = to_dev(sB), *dzA = to_dev(zA), *dzB = to_dev(zB);
    uint16_t* dC = to_dev(std::vector<uint16_t>((size_t)M * N, 0));
    clove::gemm_int4(dA, H(dsA), H(dzA), dB, H(dsB), H(dzB), H(dC), M, N, K);
    auto got = to_host(dC, (size_t)M * N);
    std::vector<uint16_t> ref16((size_t)M * N);
    std::vector<double> ref((size_t)M * N);
    oracle_gemm_int4_groupwise(A.data(), sA.data(), zA.data(), B.data(), sB.data(), zB.data(), ref16.data(),
                               nullptr, ref.data(), M, N, K);
    char name[64];
    std::snprintf(name, sizeof name, "gemm_int4 group-wise %dx%dx%d", M, N, K);
    compare(name, got, ref);
    // literal mode: B stride floor(N/2) (the reference's), zeros ignored
    if (N >= 2) {
        std::vector<uint8_t> Bl((size_t)K * (N / 2));
        for (auto& x : Bl) x = (uint8_t)g.integer(0, 255);
        uint8_t* dBl = to_dev(Bl);
        clove::gemm_int4_ex(dA, H(dsA), nullptr, dBl, H(dsB), nullptr, H(dC), M, N, K, CLOVE_INT4_REFERENCE_LITERAL);
        got = to_host(dC, (size_t)M * N);
        oracle_gemm_int4_literal(A.data(), sA.data(), Bl.data(), sB.data(), ref16.data(), M, N, K);
        std::snprintf(name, sizeof name, "gemm_int4 literal %dx%dx%d", M, N, K);
        compare_bits(name, got, ref16);
        (void)hipFree(dBl);
    }
    (void)hipFree(dA);
    (void)hipFree(dB);
    (void)hipFree(dsA);
    (void)hipFree(dsB);
    (void)hipFree(dzA);
    (void)hipFree(dzB);
    (void)hipFree(dC);
}

// ---- the layer's MLP on INT4 weights: gate/up + SwiGLU, down with the residual ----
void w4a16_mlp_case(int T) {
    const int H_ = 256, I = 384;  // hidden, intermediate
    Rng g(51 + T);
    auto X = rand_f16((size_t)T * H_, -1.0f, 1.0f, g);
    const int Gh = clove::cdiv(H_, clove::INT4_GROUP_SIZE), Gi = clove::cdiv(I, clove::INT4_GROUP_SIZE);
    std::vector<uint8_t> Wgu((size_t)2 * I * (H_ / 2)), Wd((size_t)H_ * (I / 2));
    for (auto& x : Wgu) x = (uint8_t)g.integer(0, 255);
    for (auto& x : Wd) x = (uint8_t)g.integer(0, 255);
    auto sgu = rand_f16((size_t)2 * I * Gh, 0.001f, 0.02f, g), sd = rand_f16((size_t)H_ * Gi, 0.001f, 0.02f, g);
    std::vector<uint16_t> zgu((size_t)2 * I * Gh), zd((size_t)H_ * Gi);
    for (auto& x : zgu) x = oracle_f32_to_f16((float)g.integer(0, 15));
    for (auto& x : zd) x = oracle_f32_to_f16((float)g.integer(0, 15));
    auto resid = rand_f16((size_t)T * H_, -1.0f, 1.0f, g);
    uint16_t *dX = to_dev(X), *dsgu = to_dev(sgu), *dzgu = to_dev(zgu), *dsd = to_dev(sd), *dzd = to_dev(zd);
    uint8_t *dWgu = to_dev(Wgu), *dWd = to_dev(Wd);
    uint16_t* dH = to_dev(std::vector<uint16_t>((size_t)T * I, 0));
    uint16_t* dY = to_dev(resid);
    clove::w4a16_swiglu(H(dX), dWgu, H(dsgu), H(dzgu), H(dH), T, I, H_);
    clove::gemm_w4a16(H(dH), dWd, H(dsd), H(dzd), H(dY), T, H_, I, 1.0f, 1.0f);  // down + residual
    auto h = to_host(dH, (size_t)T * I);
    auto y = to_host(dY, (size_t)T * H_);
    // oracle: gate and up projections (fp16-rounded), SwiGLU, then down + residual on the device's h
    std::vector<uint16_t> gate((size_t)T * I), up((size_t)T * I), href((size_t)T * I);
    oracle_w4a16(X.data(), Wgu.data(), sgu.data(), zgu.data(), nullptr, gate.data(), nullptr, T, I, H_, 1.0, 0.0);
    oracle_w4a16(X.data(), Wgu.data() + (size_t)I * (H_ / 2), sgu.data() + (size_t)I * Gh,
                 zgu.data() + (size_t)I * Gh, nullptr, up.data(), nullptr, T, I, H_, 1.0, 0.0);
    oracle_swiglu(gate.data(), up.data(), href.data(), (int64_t)T * I);
    std::vector<double> hd(href.size());
    for (size_t i = 0; i < href.size(); ++i) hd[i] = oracle_f16_to_f32(href[i]);
    char name[64];
    std::snprintf(name, sizeof name, "w4a16_swiglu T=%d", T);
    compare(name, h, hd);
    std::vector<double> yref((size_t)T * H_);
    oracle_w4a16(h.data(), Wd.data(), sd.data(), zd.data(), resid.data(), nullptr, yref.data(), T, H_, I, 1.0, 1.0);
    std::snprintf(name, sizeof name, "gemm_w4a16 down+residual T=%d", T);
    compare(name, y, yref);
    for (void* p : {(void*)dX, (void*)dsgu, (void*)dzgu, (void*)dsd, (void*)dzd, (void*)dWgu, (void*)dWd, (void*)dH,
                    (void*)dY})
        (void)hipFree(p);
}

void swiglu_case() {
    const int n = 10007;
    Rng g(61);
    auto gate = rand_f16(n, -8.0f, 8.0f, g), up = rand_f16(n, -2.0f, 2.0f, g);
    uint16_t *dg = to_dev(gate), *du = to_dev(up), *dout = to_dev(std::vector<uint16_t>(n, 0));
    clove::swiglu(H(dg), H(du), H(dout), n);
    auto got = to_host(dout, n);
    std::vector<uint16_t> ref(n);
    oracle_swiglu(gate.data(), up.data(), ref.data(), n);
    // device expf and libm expf may differ in the last fp32 bit: allow one fp16 ulp
    size_t bad = 0;
    for (int i = 0; i < n; ++i) {
        const int a = got[i] & 0x8000 ? -(got[i] & 0x7fff) : got[i];
        const int b = ref[i] & 0x8000 ? -(ref[i] & 0x7fff) : ref[i];
        bad += std::abs(a - b) > 1;
    }
    std::printf("%-34s %s  (%zu of %d beyond one ulp)\n", "swiglu 10007", bad ? "FAIL" : "PASS", bad, n);
    if (bad) ++g_failed;
    (void)hipFree(dg);
    (void)hipFree(du);
    (void)hipFree(dout);
}

}  // namespace

int main() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        std::fprintf(stderr, "no HIP device\n");
        return 2;
    }
    std::printf("clove C ABI version %d\n", clove_abi_version());
    // the reference header's types and constants, as its callers spell them
    static_assert(clove::CudaType<half>::dtype == clove::DType::FP16, "CudaType<half>");
    static_assert(clove::GemmConfig::NUM_THREADS == 64 * (clove::GemmConfig::BM / clove::GemmConfig::WM) *
                                                        (clove::GemmConfig::BN / clove::GemmConfig::WN),
                  "GemmConfig: one 64-lane wave per wave tile");
    if (clove::dtype_size(clove::DType::FP32) != 4 || clove::dtype_size(clove::DType::FP16) != 2 ||
        clove::dtype_size(clove::DType::BF16) != 2 || clove::dtype_size(clove::DType::INT8) != 1 ||
        clove::dtype_size(clove::DType::INT4) != 0) {
        std::printf("dtype_size FAIL\n");
        ++g_failed;
    }
    std::printf("GemmConfig %dx%dx%d, %d threads\n", clove::GemmConfig::BM, clove::GemmConfig::BN,
                clove::GemmConfig::BK, clove::GemmConfig::NUM_THREADS);
    fp16_case("test_gemm_small 64^3", 64, 64, 64, 1.0f, 0.0f, 1);
    fp16_case("test_gemm_medium 256^3", 256, 256, 256, 1.0f, 0.0f, 2);
    fp16_case("test_gemm_large 1024^3", 1024, 1024, 1024, 1.0f, 0.0f, 3);
    fp16_case("test_gemm_nonsquare 128x4096x4096", 128, 4096, 4096, 1.0f, 0.0f, 4);
    fp16_case("test_gemm_decode 1x4096x4096", 1, 4096, 4096, 1.0f, 0.0f, 5);
    fp16_case("test_gemm_alpha_beta 128^3 (0.5, 0.25)", 128, 128, 128, 0.5f, 0.25f, 6);
    fp16_default_args_case();
    batched_case();
    int8_case(64, 64, 64);
    int8_case(130, 200, 300);
    int4_case(256, 16, 1024);
    int4_case(300, 1, 4096);
    int4_case(200, 128, 512);
    swiglu_case();
    w4a16_mlp_case(1);
    w4a16_mlp_case(40);
    std::printf(g_failed ? "%d case(s) FAILED\n" : "all cases passed\n", g_failed);
    return g_failed ? 1 : 0;
}
