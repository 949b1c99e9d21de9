// C ABI of the gfx950 GEMM library: argument validation, per-stream scratch,
// dispatch to the kernel launchers.  Declarations and the reference interface
// each entry point replaces: include/clove/gemm_c.h.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <tuple>
#include <utility>
#include <vector>

#include "clove/gemm_c.h"
#include "common.hpp"
#include "dispatch.hpp"

namespace clove {
using hw::cdiv64;
namespace {

constexpr int kAbiVersion = 1;

// ---------------------------------------------------------------------------
// device info (cached per device)
// ---------------------------------------------------------------------------
std::mutex g_dev_mu;
std::map<int, int> g_num_cus;

// ---------------------------------------------------------------------------
// scratch per (device, stream)
// ---------------------------------------------------------------------------
struct ScratchEntry {
    void* base = nullptr;
    Scratch view;
};
std::mutex g_scratch_mu;
std::map<std::pair<int, void*>, ScratchEntry> g_scratch;

// other library buffers per (device, stream, slot)
struct BufferEntry {
    void* base = nullptr;
    size_t bytes = 0;
};
std::map<std::tuple<int, void*, int>, BufferEntry> g_buffers;  // guarded by g_scratch_mu

// Buffers replaced by larger ones, per device, freed by clove_release_scratch
// (after a device synchronize).  A replaced buffer is not freed on the spot: a
// call on another host thread may have taken it and not yet launched the
// kernel that uses it.  Sizes grow by powers of two, so the retired buffers
// of a stream add up to less than its current one.
std::map<int, std::vector<void*>> g_retired;  // guarded by g_scratch_mu

__global__ void zero_u16(uint16_t* p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

__global__ void zero_u32(unsigned* p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

size_t round_up_pow2(size_t x, size_t floor_bytes) {
    size_t r = floor_bytes;
    while (r < x) r <<= 1;
    return r;
}

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
    if (!a || !b || abytes == 0 || bbytes == 0) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + bbytes && b0 < a0 + abytes;
}

bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace

clove_status_t ensure_lds(const void* kernel, int bytes) {
    if (bytes <= 64 * 1024) return CLOVE_OK;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    static std::mutex mu;
    static std::vector<std::tuple<int, const void*, int>> done;  // (device, kernel, bytes set)
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& e : done)
        if (std::get<0>(e) == dev && std::get<1>(e) == kernel && std::get<2>(e) >= bytes) return CLOVE_OK;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
        return CLOVE_ERR_LAUNCH;
    done.emplace_back(dev, kernel, bytes);
    return CLOVE_OK;
}

namespace {

// ---------------------------------------------------------------------------
// caller-owned workspace (clove_workspace_bind / clove_workspace_query_*), per
// host thread.  Layout of a bound workspace: the completion counters at its
// start (a fixed region, so a counter never lands where an earlier call left
// partial sums), then each acquisition of the call at 256-byte offsets.
// ---------------------------------------------------------------------------
enum class WsMode { kLibrary, kBound, kQuery };
struct ThreadWs {
    WsMode mode = WsMode::kLibrary;
    char* ptr = nullptr;
    size_t bytes = 0;
    size_t used = 0;  // carve offset of the current call
    size_t need = 0;  // query: the largest call so far
};
thread_local ThreadWs t_ws;
thread_local ThreadWs t_ws_saved;  // the mode a query interrupted
constexpr size_t kWsCounterBytes = CLOVE_WORKSPACE_MIN_BYTES;
constexpr size_t kWsCounters = kWsCounterBytes / sizeof(unsigned);

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Carves `bytes` for the current call; nullptr-based in a query (nothing is
// launched, so nothing reads it).
clove_status_t ws_carve(size_t bytes, char** out) {
    const size_t off = t_ws.used;
    t_ws.used += round256(bytes);
    if (t_ws.mode == WsMode::kBound && t_ws.used > t_ws.bytes) return CLOVE_ERR_WORKSPACE;
    *out = reinterpret_cast<char*>(reinterpret_cast<uintptr_t>(t_ws.ptr) + off);
    return CLOVE_OK;
}

// One per C entry point that dispatches: starts the call's carving after the
// counters and, in a query, records what the call took.
struct CallScope {
    CallScope() { t_ws.used = kWsCounterBytes; }
    ~CallScope() {
        if (t_ws.mode == WsMode::kQuery && t_ws.used > kWsCounterBytes && t_ws.used > t_ws.need)
            t_ws.need = t_ws.used;
    }
};

// ---------------------------------------------------------------------------
// clove_gemm_fp16_noalloc: the fixed device array its calls carve their
// scratch from (counters in its first CLOVE_WORKSPACE_MIN_BYTES, as in a bound
// workspace).  In host code `scratch` is a host-side stand-in for the symbol,
// not a device address: the address each device holds its copy at comes from
// hipGetSymbolAddress, once per device, and only that address is used.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocBytes = CLOVE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];
std::mutex g_noalloc_mu;
std::map<int, char*> g_noalloc_ptr;  // device -> address of its `scratch`

clove_status_t noalloc_scratch(hipStream_t stream, char** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    auto it = g_noalloc_ptr.find(dev);
    if (it == g_noalloc_ptr.end()) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
            return CLOVE_ERR_NO_DEVICE;
        // the counters start at zero (every call leaves them zero again)
        hipLaunchKernelGGL(zero_u32, dim3(16), dim3(256), 0, stream, static_cast<unsigned*>(ptr), kWsCounters);
        if (hipGetLastError() != hipSuccess) return CLOVE_ERR_LAUNCH;
        it = g_noalloc_ptr.emplace(dev, static_cast<char*>(ptr)).first;
    }
    *out = it->second;
    return CLOVE_OK;
}

}  // namespace

bool dry_run() { return t_ws.mode == WsMode::kQuery; }

clove_status_t current_device_info(DeviceInfo* out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    auto it = g_num_cus.find(dev);
    if (it == g_num_cus.end()) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            return CLOVE_ERR_NO_DEVICE;
        it = g_num_cus.emplace(dev, cus).first;
    }
    out->device = dev;
    out->num_cus = it->second;
    return CLOVE_OK;
}

clove_status_t acquire_scratch(hipStream_t stream, size_t partial_bytes, size_t num_counters,
                               Scratch* out) {
    if (t_ws.mode != WsMode::kLibrary) {
        if (num_counters > kWsCounters) return CLOVE_ERR_WORKSPACE;
        char* part = nullptr;
        const clove_status_t st = ws_carve(partial_bytes, &part);
        if (st != CLOVE_OK) return st;
        out->partials = reinterpret_cast<float*>(part);
        out->partial_bytes = round256(partial_bytes);
        out->counters = reinterpret_cast<unsigned*>(t_ws.ptr);
        out->num_counters = kWsCounters;
        return CLOVE_OK;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ScratchEntry& e = g_scratch[{dev, reinterpret_cast<void*>(stream)}];
    if (e.base && e.view.partial_bytes >= partial_bytes && e.view.num_counters >= num_counters) {
        *out = e.view;
        return CLOVE_OK;
    }
    const size_t pb = round_up_pow2(partial_bytes, (size_t)4 << 20);
    const size_t nc = round_up_pow2(num_counters, 4096);
    void* base = nullptr;
    if (hipMalloc(&base, pb + nc * sizeof(unsigned)) != hipSuccess) return CLOVE_ERR_OUT_OF_MEMORY;
    if (e.base) {
        // queued work (and calls of other host threads) may still use the old buffer
        g_retired[dev].push_back(e.base);
        e = ScratchEntry{};
    }
    unsigned* counters = reinterpret_cast<unsigned*>(static_cast<char*>(base) + pb);
    hipLaunchKernelGGL(zero_u32, dim3(64), dim3(256), 0, stream, counters, nc);
    if (hipGetLastError() != hipSuccess) {
        (void)hipFree(base);
        return CLOVE_ERR_LAUNCH;
    }
    e.base = base;
    e.view.partials = static_cast<float*>(base);
    e.view.partial_bytes = pb;
    e.view.counters = counters;
    e.view.num_counters = nc;
    *out = e.view;
    return CLOVE_OK;
}

clove_status_t acquire_buffer(hipStream_t stream, int slot, size_t bytes, void** out) {
    if (t_ws.mode != WsMode::kLibrary) {
        char* p = nullptr;
        const clove_status_t st = ws_carve(bytes, &p);
        *out = p;
        return st;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    BufferEntry& e = g_buffers[std::make_tuple(dev, reinterpret_cast<void*>(stream), slot)];
    if (e.base && e.bytes >= bytes) {
        *out = e.base;
        return CLOVE_OK;
    }
    const size_t nb = round_up_pow2(bytes, (size_t)1 << 20);
    void* base = nullptr;
    if (hipMalloc(&base, nb) != hipSuccess) return CLOVE_ERR_OUT_OF_MEMORY;
    if (e.base) g_retired[dev].push_back(e.base);  // as in acquire_scratch
    e.base = base;
    e.bytes = nb;
    *out = e.base;
    return CLOVE_OK;
}

}  // namespace clove

using namespace clove;

extern "C" {

const char* clove_status_string(clove_status_t status) {
    switch (status) {
        case CLOVE_OK: return "CLOVE_OK";
        case CLOVE_ERR_NULL_POINTER: return "CLOVE_ERR_NULL_POINTER: a required pointer is NULL";
        case CLOVE_ERR_INVALID_DIM: return "CLOVE_ERR_INVALID_DIM: a dimension is negative or too large";
        case CLOVE_ERR_INVALID_ARG: return "CLOVE_ERR_INVALID_ARG: invalid argument (odd K for INT4, mode, alignment)";
        case CLOVE_ERR_ALIASING: return "CLOVE_ERR_ALIASING: output overlaps an input";
        case CLOVE_ERR_OUT_OF_MEMORY: return "CLOVE_ERR_OUT_OF_MEMORY: scratch allocation failed";
        case CLOVE_ERR_LAUNCH: return "CLOVE_ERR_LAUNCH: kernel launch failed";
        case CLOVE_ERR_NO_DEVICE: return "CLOVE_ERR_NO_DEVICE: no usable HIP device";
        case CLOVE_ERR_WORKSPACE: return "CLOVE_ERR_WORKSPACE: the bound workspace is too small for the call";
        case CLOVE_ERR_SCRATCH_LIMIT:
            return "CLOVE_ERR_SCRATCH_LIMIT: the call needs more scratch than the fixed array of "
                   "clove_gemm_fp16_noalloc holds (CLOVE_NOALLOC_SCRATCH_BYTES)";
    }
    return "CLOVE_ERR_UNKNOWN";
}

int clove_abi_version(void) { return kAbiVersion; }

clove_status_t clove_gemm_fp16_batched(const void* A, const void* B, void* C, int batch, int M,
                                       int N, int K, float alpha, float beta, void* stream) {
    CallScope scope;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return CLOVE_ERR_INVALID_DIM;
    if (batch == 0 || M == 0 || N == 0) return CLOVE_OK;
    if (!C || (K > 0 && (!A || !B))) return CLOVE_ERR_NULL_POINTER;
    if (!aligned2(A) || !aligned2(B) || !aligned2(C)) return CLOVE_ERR_INVALID_ARG;
    const size_t bc = (size_t)batch * M * N * 2;
    if (overlaps(C, bc, A, (size_t)batch * M * K * 2) || overlaps(C, bc, B, (size_t)batch * K * N * 2))
        return CLOVE_ERR_ALIASING;
    if ((int64_t)batch * (int64_t)cdiv64(M, 32) * (int64_t)cdiv64(N, 128) > 0x3fffffff)
        return CLOVE_ERR_INVALID_DIM;
    return launch_gemm_fp16(static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B),
                            static_cast<uint16_t*>(C), batch, M, N, K, alpha, beta,
                            static_cast<hipStream_t>(stream));
}

clove_status_t clove_gemm_fp16(const void* A, const void* B, void* C, int M, int N, int K,
                               float alpha, float beta, void* stream) {
    return clove_gemm_fp16_batched(A, B, C, 1, M, N, K, alpha, beta, stream);
}

clove_status_t clove_gemm_fp16_noalloc(const void* A, const void* B, void* C, int M, int N, int K,
                                       float alpha, float beta, void* stream) {
    if (t_ws.mode == WsMode::kQuery) {
        // plan and validate as clove_gemm_fp16, and report a call the fixed
        // array cannot hold as the real call would; the array is not the
        // caller's workspace, so the query's size is left as it was
        const size_t need = t_ws.need;
        t_ws.need = 0;
        clove_status_t st = clove_gemm_fp16(A, B, C, M, N, K, alpha, beta, stream);
        if (st == CLOVE_OK && t_ws.need > kNoAllocBytes) st = CLOVE_ERR_SCRATCH_LIMIT;
        t_ws.need = need;
        return st;
    }
    char* ptr = nullptr;
    clove_status_t st = noalloc_scratch(static_cast<hipStream_t>(stream), &ptr);
    if (st != CLOVE_OK) return st;
    // the call runs with this thread's workspace bound to the array, then the
    // thread's own mode is restored
    const ThreadWs saved = t_ws;
    t_ws = ThreadWs{};
    t_ws.mode = WsMode::kBound;
    t_ws.ptr = ptr;
    t_ws.bytes = kNoAllocBytes;
    st = clove_gemm_fp16(A, B, C, M, N, K, alpha, beta, stream);
    t_ws = saved;
    return st == CLOVE_ERR_WORKSPACE ? CLOVE_ERR_SCRATCH_LIMIT : st;
}

static clove_status_t int8_common(Int8Args& a, void* stream) {
    CallScope scope;
    if (a.M < 0 || a.N < 0 || a.K < 0) return CLOVE_ERR_INVALID_DIM;
    if (a.M == 0 || a.N == 0) return CLOVE_OK;
    if (!a.C || (a.K > 0 && (!a.A || !a.B))) return CLOVE_ERR_NULL_POINTER;
    const size_t out_elt = a.out == Int8Out::kAcc32 ? 4 : 2;
    if (a.out == Int8Out::kAcc32 ? (reinterpret_cast<uintptr_t>(a.C) & 3u) != 0 : !aligned2(a.C))
        return CLOVE_ERR_INVALID_ARG;
    const size_t bc = (size_t)a.M * a.N * out_elt;
    if (overlaps(a.C, bc, a.A, (size_t)a.M * a.K) || overlaps(a.C, bc, a.B, (size_t)a.K * a.N))
        return CLOVE_ERR_ALIASING;
    if (a.out == Int8Out::kHalfRowCol) {
        if (!a.sa || !a.sb) return CLOVE_ERR_NULL_POINTER;
        if (!aligned2(a.sa) || !aligned2(a.sb)) return CLOVE_ERR_INVALID_ARG;
        if (overlaps(a.C, bc, a.sa, (size_t)a.M * 2) || overlaps(a.C, bc, a.sb, (size_t)a.N * 2))
            return CLOVE_ERR_ALIASING;
    }
    return launch_gemm_int8(a, static_cast<hipStream_t>(stream));
}

clove_status_t clove_gemm_int8(const int8_t* A_q, const int8_t* B_q, void* C, int M, int N, int K,
                               float A_scale, int8_t A_zero, float B_scale, int8_t B_zero,
                               void* stream) {
    Int8Args a;
    a.A = A_q; a.B = B_q; a.C = C; a.M = M; a.N = N; a.K = K;
    a.scale = A_scale * B_scale;  // combined in fp32 (src/kernels/gemm_int8.cu:40)
    a.za = A_zero; a.zb = B_zero;
    a.out = Int8Out::kHalfPerTensor;
    return int8_common(a, stream);
}

clove_status_t clove_gemm_int8_ex(const int8_t* A_q, const int8_t* B_q, void* C, int M, int N, int K,
                                  float A_scale, int8_t A_zero, float B_scale, int8_t B_zero, int mode,
                                  void* stream) {
    if (mode != CLOVE_INT8_EXACT && mode != CLOVE_INT8_REFERENCE_LITERAL) return CLOVE_ERR_INVALID_ARG;
    Int8Args a;
    a.A = A_q; a.B = B_q; a.C = C; a.M = M; a.N = N; a.K = K;
    a.scale = A_scale * B_scale;  // combined in fp32 (src/kernels/gemm_int8.cu:40)
    a.za = A_zero; a.zb = B_zero;
    if (mode == CLOVE_INT8_REFERENCE_LITERAL && K > 0) {
        // the reference walks K in 32-wide tiles, loads 0 past K and subtracts
        // the zero points from it (src/kernels/gemm_int8.cu:43, 52-54, 63-64,
        // 89-93): each padded k adds za * zb
        const unsigned pad = (unsigned)(32 * ((K + 31) / 32) - K);
        a.acc_add = (int)(pad * (unsigned)(int)A_zero * (unsigned)(int)B_zero);
    }
    a.out = Int8Out::kHalfPerTensor;
    return int8_common(a, stream);
}

clove_status_t clove_gemm_int8_rowcol(const int8_t* A_q, const int8_t* B_q, const void* A_scale,
                                      const void* B_scale, void* C, int M, int N, int K,
                                      int8_t A_zero, int8_t B_zero, void* stream) {
    Int8Args a;
    a.A = A_q; a.B = B_q; a.C = C; a.M = M; a.N = N; a.K = K;
    a.sa = static_cast<const uint16_t*>(A_scale);
    a.sb = static_cast<const uint16_t*>(B_scale);
    a.za = A_zero; a.zb = B_zero;
    a.out = Int8Out::kHalfRowCol;
    return int8_common(a, stream);
}

clove_status_t clove_gemm_int8_acc32(const int8_t* A_q, const int8_t* B_q, int32_t* acc, int M,
                                     int N, int K, int8_t A_zero, int8_t B_zero, void* stream) {
    Int8Args a;
    a.A = A_q; a.B = B_q; a.C = acc; a.M = M; a.N = N; a.K = K;
    a.za = A_zero; a.zb = B_zero;
    a.out = Int8Out::kAcc32;
    return int8_common(a, stream);
}

clove_status_t clove_gemm_int4_ex(const uint8_t* A_q, const void* A_scale, const void* A_zero,
                                  const uint8_t* B_q, const void* B_scale, const void* B_zero,
                                  void* C, int M, int N, int K, clove_int4_mode_t mode,
                                  void* stream) {
    CallScope scope;
    if (mode != CLOVE_INT4_GROUPWISE && mode != CLOVE_INT4_REFERENCE_LITERAL)
        return CLOVE_ERR_INVALID_ARG;
    if (M < 0 || N < 0 || K < 0) return CLOVE_ERR_INVALID_DIM;
    if (K % 2 != 0) return CLOVE_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return CLOVE_OK;
    const bool literal = mode == CLOVE_INT4_REFERENCE_LITERAL;
    if (!C) return CLOVE_ERR_NULL_POINTER;
    if (K > 0) {
        if (!A_q || !A_scale || !B_scale) return CLOVE_ERR_NULL_POINTER;
        if (!literal && (!A_zero || !B_zero || !B_q)) return CLOVE_ERR_NULL_POINTER;
        if (literal && N >= 2 && !B_q) return CLOVE_ERR_NULL_POINTER;
    }
    if (!aligned2(C) || !aligned2(A_scale) || !aligned2(B_scale) || !aligned2(A_zero) ||
        !aligned2(B_zero))
        return CLOVE_ERR_INVALID_ARG;
    const int64_t G = cdiv64(K, 128);
    const size_t bc = (size_t)M * N * 2;
    const size_t bstride = literal ? (size_t)(N / 2) : (size_t)((N + 1) / 2);
    if (overlaps(C, bc, A_q, (size_t)M * (K / 2)) || overlaps(C, bc, B_q, (size_t)K * bstride) ||
        overlaps(C, bc, A_scale, (size_t)M * G * 2) || overlaps(C, bc, B_scale, (size_t)G * N * 2) ||
        (!literal && (overlaps(C, bc, A_zero, (size_t)M * G * 2) ||
                      overlaps(C, bc, B_zero, (size_t)G * N * 2))))
        return CLOVE_ERR_ALIASING;
    Int4Args a;
    a.A = A_q;
    a.A_scale = static_cast<const uint16_t*>(A_scale);
    a.A_zero = static_cast<const uint16_t*>(A_zero);
    a.B = B_q;
    a.B_scale = static_cast<const uint16_t*>(B_scale);
    a.B_zero = static_cast<const uint16_t*>(B_zero);
    a.C = static_cast<uint16_t*>(C);
    a.M = M; a.N = N; a.K = K;
    a.mode = mode;
    return launch_gemm_int4(a, static_cast<hipStream_t>(stream));
}

clove_status_t clove_gemm_int4(const uint8_t* A_q, const void* A_scale, const void* A_zero,
                               const uint8_t* B_q, const void* B_scale, const void* B_zero,
                               void* C, int M, int N, int K, void* stream) {
    return clove_gemm_int4_ex(A_q, A_scale, A_zero, B_q, B_scale, B_zero, C, M, N, K,
                              CLOVE_INT4_GROUPWISE, stream);
}

clove_status_t clove_gemm_int4_group_acc32(const uint8_t* A_q, const void* A_zero, const uint8_t* B_q,
                                           const void* B_zero, int32_t* P, int M, int N, int K,
                                           void* stream) {
    CallScope scope;
    if (M < 0 || N < 0 || K < 0) return CLOVE_ERR_INVALID_DIM;
    if (M == 0 || N == 0 || K == 0) return CLOVE_OK;
    if (!A_q || !A_zero || !B_q || !B_zero || !P) return CLOVE_ERR_NULL_POINTER;
    if (K % 256 != 0 || !aligned16(A_q) || !aligned4(P) || !aligned2(A_zero) || !aligned2(B_zero))
        return CLOVE_ERR_INVALID_ARG;
    const int64_t G = K / 128;
    const size_t bp = (size_t)M * N * G * 4;
    if (overlaps(P, bp, A_q, (size_t)M * (K / 2)) || overlaps(P, bp, B_q, (size_t)K * ((N + 1) / 2)) ||
        overlaps(P, bp, A_zero, (size_t)M * G * 2) || overlaps(P, bp, B_zero, (size_t)G * N * 2))
        return CLOVE_ERR_ALIASING;
    DeviceInfo dev;
    clove_status_t st = current_device_info(&dev);
    if (st != CLOVE_OK) return st;
    Int4Args a;
    a.A = A_q;
    a.A_zero = static_cast<const uint16_t*>(A_zero);
    a.B = B_q;
    a.B_zero = static_cast<const uint16_t*>(B_zero);
    a.M = M; a.N = N; a.K = K;
    return launch_i4i4_partials(a, P, dev.num_cus, static_cast<hipStream_t>(stream));
}

clove_status_t clove_gemm_w4a16(const void* X, const uint8_t* W_q, const void* W_scale,
                                const void* W_zero, void* Y, int T, int O, int K, float alpha,
                                float beta, void* stream) {
    CallScope scope;
    if (T < 0 || O < 0 || K < 0) return CLOVE_ERR_INVALID_DIM;
    if (K % 2 != 0) return CLOVE_ERR_INVALID_ARG;
    if (T == 0 || O == 0) return CLOVE_OK;
    if (!Y || (K > 0 && (!X || !W_q || !W_scale || !W_zero))) return CLOVE_ERR_NULL_POINTER;
    if (!aligned2(X) || !aligned2(Y) || !aligned2(W_scale) || !aligned2(W_zero))
        return CLOVE_ERR_INVALID_ARG;
    const int64_t G = cdiv64(K, 128);
    const size_t by = (size_t)T * O * 2;
    if (overlaps(Y, by, X, (size_t)T * K * 2) || overlaps(Y, by, W_q, (size_t)O * (K / 2)) ||
        overlaps(Y, by, W_scale, (size_t)O * G * 2) || overlaps(Y, by, W_zero, (size_t)O * G * 2))
        return CLOVE_ERR_ALIASING;
    W4A16Args a;
    a.X = static_cast<const uint16_t*>(X);
    a.W = W_q;
    a.scale = static_cast<const uint16_t*>(W_scale);
    a.zero = static_cast<const uint16_t*>(W_zero);
    a.Y = static_cast<uint16_t*>(Y);
    a.T = T; a.O = O; a.K = K;
    a.alpha = alpha; a.beta = beta;
    return launch_w4a16(a, static_cast<hipStream_t>(stream));
}

static bool same_or_disjoint(const void* a, const void* b, size_t bytes) {
    return a == b || !overlaps(a, bytes, b, bytes);
}

clove_status_t clove_swiglu(const void* gate, const void* up, void* output, int size, void* stream) {
    CallScope scope;
    if (size < 0) return CLOVE_ERR_INVALID_DIM;
    if (size == 0) return CLOVE_OK;
    if (!gate || !up || !output) return CLOVE_ERR_NULL_POINTER;
    if (!aligned2(gate) || !aligned2(up) || !aligned2(output)) return CLOVE_ERR_INVALID_ARG;
    // elementwise: the output may be one of the inputs, but not shifted against it
    const size_t b = (size_t)size * 2;
    if (!same_or_disjoint(output, gate, b) || !same_or_disjoint(output, up, b)) return CLOVE_ERR_ALIASING;
    return launch_swiglu(static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                         static_cast<uint16_t*>(output), size, static_cast<hipStream_t>(stream));
}

clove_status_t clove_swiglu_fused(const void* input, const void* W_gate, const void* W_up, void* output,
                                  int batch_seq, int hidden_dim, int intermediate_dim, void* stream) {
    CallScope scope;
    const int T = batch_seq, H = hidden_dim, I = intermediate_dim;
    if (T < 0 || H < 0 || I < 0) return CLOVE_ERR_INVALID_DIM;
    if (T == 0 || I == 0) return CLOVE_OK;
    if (!output || (H > 0 && (!input || !W_gate || !W_up))) return CLOVE_ERR_NULL_POINTER;
    if (!aligned2(input) || !aligned2(W_gate) || !aligned2(W_up) || !aligned2(output))
        return CLOVE_ERR_INVALID_ARG;
    const size_t bo = (size_t)T * I * 2;
    if (overlaps(output, bo, input, (size_t)T * H * 2) || overlaps(output, bo, W_gate, (size_t)H * I * 2) ||
        overlaps(output, bo, W_up, (size_t)H * I * 2))
        return CLOVE_ERR_ALIASING;
    if ((int64_t)cdiv64(T, 32) * (int64_t)cdiv64(I, 128) > 0x3fffffff) return CLOVE_ERR_INVALID_DIM;
    return launch_swiglu_fused_fp16(static_cast<const uint16_t*>(input), static_cast<const uint16_t*>(W_gate),
                                    static_cast<const uint16_t*>(W_up), static_cast<uint16_t*>(output), T, H,
                                    I, static_cast<hipStream_t>(stream));
}

clove_status_t clove_w4a16_swiglu(const void* X, const uint8_t* W_q, const void* W_scale,
                                  const void* W_zero, void* H, int T, int I, int K, void* stream) {
    CallScope scope;
    if (T < 0 || I < 0 || K < 0) return CLOVE_ERR_INVALID_DIM;
    if (K % 2 != 0) return CLOVE_ERR_INVALID_ARG;
    if (T == 0 || I == 0) return CLOVE_OK;
    if (!H || (K > 0 && (!X || !W_q || !W_scale || !W_zero))) return CLOVE_ERR_NULL_POINTER;
    if (!aligned2(X) || !aligned2(H) || !aligned2(W_scale) || !aligned2(W_zero)) return CLOVE_ERR_INVALID_ARG;
    if ((int64_t)2 * I > 0x7fffffff) return CLOVE_ERR_INVALID_DIM;
    const int64_t G = cdiv64(K, 128);
    const size_t bh = (size_t)T * I * 2;
    if (overlaps(H, bh, X, (size_t)T * K * 2) || overlaps(H, bh, W_q, (size_t)2 * I * (K / 2)) ||
        overlaps(H, bh, W_scale, (size_t)2 * I * G * 2) || overlaps(H, bh, W_zero, (size_t)2 * I * G * 2))
        return CLOVE_ERR_ALIASING;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (K == 0) {  // gate = up = 0: swiglu(0, 0) = +0
        CLOVE_LAUNCH(zero_u16, dim3(256), dim3(256), 0, s, static_cast<uint16_t*>(H), (size_t)T * I);
        return check_launch();
    }
    W4A16Args a;
    a.X = static_cast<const uint16_t*>(X);
    a.W = W_q;
    a.scale = static_cast<const uint16_t*>(W_scale);
    a.zero = static_cast<const uint16_t*>(W_zero);
    a.Y = static_cast<uint16_t*>(H);
    a.T = T; a.O = I; a.K = K;
    return launch_w4a16_swiglu(a, s);
}

clove_status_t clove_workspace_bind(void* ptr, size_t bytes) {
    if (t_ws.mode == WsMode::kQuery) return CLOVE_ERR_INVALID_ARG;
    if (!ptr) {
        if (bytes != 0) return CLOVE_ERR_NULL_POINTER;
        t_ws = ThreadWs{};
        return CLOVE_OK;
    }
    if ((reinterpret_cast<uintptr_t>(ptr) & 255u) != 0) return CLOVE_ERR_INVALID_ARG;
    if (bytes < kWsCounterBytes) return CLOVE_ERR_WORKSPACE;
    t_ws = ThreadWs{};
    t_ws.mode = WsMode::kBound;
    t_ws.ptr = static_cast<char*>(ptr);
    t_ws.bytes = bytes;
    return CLOVE_OK;
}

clove_status_t clove_workspace_query_begin(void) {
    if (t_ws.mode == WsMode::kQuery) return CLOVE_ERR_INVALID_ARG;
    t_ws_saved = t_ws;
    t_ws = ThreadWs{};
    t_ws.mode = WsMode::kQuery;
    return CLOVE_OK;
}

size_t clove_workspace_query_end(void) {
    if (t_ws.mode != WsMode::kQuery) return 0;
    const size_t need = t_ws.need;
    t_ws = t_ws_saved;
    t_ws_saved = ThreadWs{};
    return need;
}

clove_status_t clove_release_scratch(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CLOVE_ERR_NO_DEVICE;
    if (hipDeviceSynchronize() != hipSuccess) return CLOVE_ERR_LAUNCH;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    for (auto it = g_scratch.begin(); it != g_scratch.end();) {
        if (it->first.first == dev) {
            (void)hipFree(it->second.base);
            it = g_scratch.erase(it);
        } else {
            ++it;
        }
    }
    for (auto it = g_buffers.begin(); it != g_buffers.end();) {
        if (std::get<0>(it->first) == dev) {
            (void)hipFree(it->second.base);
            it = g_buffers.erase(it);
        } else {
            ++it;
        }
    }
    for (void* p : g_retired[dev]) (void)hipFree(p);
    g_retired.erase(dev);
    return CLOVE_OK;
}

}  // extern "C"
