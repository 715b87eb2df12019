// The reference's ten legacy exports (engine/native_quant.cpp:705-768), same
// names, argument order and host-pointer semantics, backed by the GPU kernels.
//
// raw is GGML bytes in host memory (a GGUF mmap slice in the reference,
// engine/gguf_parser.py:153-156). Uploading and repacking 33 MB per call
// would dominate, so a call whose raw lies inside a range declared immutable
// with localai_hip_register_host() (or any call when LOCALAI_HIP_ASSUME_IMMUTABLE=1)
// reuses a device copy keyed by (address, type, rows, cols). Other calls
// upload into a temporary copy. Calls are serialised by one mutex, as the
// reference serialises its pool (engine/native_quant.cpp:361-363).
//
// x goes up through a pinned host staging buffer (hipHostMalloc, grown on
// demand) with an asynchronous copy on the library's legacy stream; the
// matvecs store the result straight into a second pinned buffer (host memory
// the device addresses: 30.0 -> 22.1 us per Q4_K 14336 x 4096 call against a
// download copy; a copy kernel for x instead of the DMA copy gained nothing),
// the GEMM through an asynchronous download; a call waits once, at the end.
//
// The exports return void like the reference; a failure leaves NaN in `out`
// and the status in localai_hip_last_status().
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "internal.h"

namespace lq {
namespace {

std::mutex g_mu;
std::vector<std::pair<uintptr_t, size_t>> g_ranges;
std::map<std::tuple<uintptr_t, int, int, int>, localai_qmat *> g_cache;
float *g_x = nullptr, *g_y = nullptr, *g_ws = nullptr;
size_t g_x_cap = 0, g_y_cap = 0, g_ws_cap = 0;
float *g_hx = nullptr, *g_hy = nullptr;   // pinned host staging of x and y
size_t g_hx_cap = 0, g_hy_cap = 0;
hipStream_t g_stream = nullptr;           // the legacy calls' stream (default priority)
// tokens from which the legacy matmul runs the MFMA GEMM (f16 operands, fp32
// accumulation) instead of the fp32 matvec
constexpr int kGemmTokens = 32;

bool assume_immutable() {
    const char *e = getenv("LOCALAI_HIP_ASSUME_IMMUTABLE");
    return e && e[0] == '1';
}

bool registered(uintptr_t p, size_t n) {
    for (auto &r : g_ranges)
        if (p >= r.first && p + n <= r.first + r.second) return true;
    return false;
}

int grow(float **buf, size_t *cap, size_t n) {
    if (*cap >= n) return LOCALAI_OK;
    if (*buf) hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
    LQ_HIP(hipMalloc((void **)buf, n * sizeof(float)));
    *cap = n;
    return LOCALAI_OK;
}

int grow_pinned(float **buf, size_t *cap, size_t n) {
    if (*cap >= n) return LOCALAI_OK;
    if (*buf) hipHostFree(*buf);
    *buf = nullptr;
    *cap = 0;
    LQ_HIP(hipHostMalloc((void **)buf, n * sizeof(float), hipHostMallocDefault));
    *cap = n;
    return LOCALAI_OK;
}

// Resolve raw -> device handle; *temp is set when the caller must destroy it.
int resolve(const uint8_t *raw, int t, int rows, int cols, localai_qmat **m, bool *temp) {
    const lq_geom g = lq_make_geom(t, rows, cols, 1);
    const uintptr_t p = reinterpret_cast<uintptr_t>(raw);
    const bool cacheable = assume_immutable() || registered(p, (size_t)g.ggml_matrix_bytes);
    auto key = std::make_tuple(p, t, rows, cols);
    if (cacheable) {
        auto it = g_cache.find(key);
        if (it != g_cache.end()) {
            *m = it->second;
            *temp = false;
            return LOCALAI_OK;
        }
    }
    int st = localai_hip_qmat_create(t, rows, cols, 1, raw, 0, nullptr, m);
    if (st) return st;
    if (cacheable) g_cache[key] = *m;
    *temp = !cacheable;
    return LOCALAI_OK;
}

void fill_nan(float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = std::nanf("");
}

int validate(int t, int rows, int cols, int tokens) {
    int bv = lq_block_values(t);
    if (rows < 1 || tokens < 1 || cols < bv || cols % bv)
        return fail(LOCALAI_EARG, "rows/tokens must be >= 1 and cols a positive multiple of the block size");
    return LOCALAI_OK;
}

int run(int t, const uint8_t *raw, const float *x, float *out, int rows, int cols, int tokens,
        bool transpose_out) {
    if (int st = validate(t, rows, cols, tokens)) return st;
    if (!raw || !x || !out) return fail(LOCALAI_EARG, "null pointer");
    if (int st = ensure_device()) return st;
    localai_qmat *m = nullptr;
    bool temp = false;
    if (int st = resolve(raw, t, rows, cols, &m, &temp)) return st;
    const size_t nx = (size_t)tokens * cols, ny = (size_t)tokens * rows;
    int st = LOCALAI_OK;
    if (!g_stream) {
        hipError_t e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
        if (e != hipSuccess) st = hip_fail(e, "legacy stream");
    }
    if (!st) st = grow(&g_x, &g_x_cap, nx);
    if (!st) st = grow(&g_y, &g_y_cap, ny);
    if (!st) st = grow_pinned(&g_hx, &g_hx_cap, nx);
    if (!st) st = grow_pinned(&g_hy, &g_hy_cap, ny);
    hipStream_t s = g_stream;
    if (!st) {
        memcpy(g_hx, x, nx * 4);
        hipError_t e = hipMemcpyAsync(g_x, g_hx, nx * 4, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) st = hip_fail(e, "upload x");
    }
    // many-token calls take the MFMA GEMM and write the reference's [rows, tokens]
    // layout directly (engine/native_quant.cpp:492); fewer tokens take the matvec
    const bool gemm = transpose_out && tokens >= kGemmTokens;
    if (!st && gemm) {
        const int64_t wsb = gemm_workspace_bytes(m->g, tokens);
        st = grow(&g_ws, &g_ws_cap, (size_t)(wsb + 3) / 4);
        if (!st) st = launch_gemm(m->g, m->tiles ? nullptr : m->data, m->tiles, g_x, tokens, g_y, 1, tokens, g_ws, wsb,
                                  s);
    } else if (!st) {
        // the matvecs store y straight into the pinned staging buffer (host
        // memory the device can address): no download copy
        if (m->tiles && tokens == 1 && mt_matvec_ok(m->g)) {
            st = launch_matvec_mfma(m->g, m->tiles, g_x, g_hy, s);
        } else if (m->tiles && mt_matvec_ok(m->g)) {
            st = launch_matvec_mfma_tok(m->g, m->tiles, g_x, cols, g_hy, rows, tokens, s);
        } else {
            const uint8_t *planes = qmat_planes(m, s, &st);
            if (planes) st = launch_matvec(m->g, planes, g_x, cols, g_hy, rows, tokens, s);
        }
    }
    if (!st) {
        hipError_t e = gemm ? hipMemcpyAsync(g_hy, g_y, ny * 4, hipMemcpyDeviceToHost, s) : hipSuccess;
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) st = hip_fail(e, "download y");
    }
    if (!st) {
        if (!transpose_out || gemm) {
            memcpy(out, g_hy, ny * 4);
        } else {
            // reference matmul output is [rows, tokens] (engine/native_quant.cpp:492)
            for (int tk = 0; tk < tokens; ++tk)
                for (int r = 0; r < rows; ++r) out[(size_t)r * tokens + tk] = g_hy[(size_t)tk * rows + r];
        }
    }
    if (st && g_stream) (void)hipStreamSynchronize(g_stream);   // nothing of this call left in flight
    if (temp) localai_hip_qmat_destroy(m);
    return st;
}

void legacy(int t, const uint8_t *raw, const float *x, float *out, int rows, int cols, int tokens,
            bool matmul) {
    std::lock_guard<std::mutex> lk(g_mu);
    clear_error();
    int st = run(t, raw, x, out, rows, cols, tokens, matmul);
    set_legacy_status(st);
    if (st && out && rows > 0 && tokens > 0) fill_nan(out, (size_t)rows * tokens);
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int localai_hip_register_host(const void *host, size_t nbytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    clear_error();
    if (!host || nbytes == 0) return fail(LOCALAI_EARG, "empty range");
    g_ranges.emplace_back(reinterpret_cast<uintptr_t>(host), nbytes);
    return LOCALAI_OK;
}

int localai_hip_unregister_host(const void *host) {
    std::lock_guard<std::mutex> lk(g_mu);
    clear_error();
    const uintptr_t p = reinterpret_cast<uintptr_t>(host);
    size_t n = 0;
    for (size_t i = 0; i < g_ranges.size(); ++i)
        if (g_ranges[i].first == p) { n = g_ranges[i].second; g_ranges.erase(g_ranges.begin() + i); break; }
    if (n == 0) return fail(LOCALAI_EARG, "range not registered");
    for (auto it = g_cache.begin(); it != g_cache.end();) {
        uintptr_t a = std::get<0>(it->first);
        if (a >= p && a < p + n) { localai_hip_qmat_destroy(it->second); it = g_cache.erase(it); }
        else ++it;
    }
    return LOCALAI_OK;
}

int64_t localai_hip_cache_entries(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return (int64_t)g_cache.size();
}

int localai_hip_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    clear_error();
    for (auto &kv : g_cache) localai_hip_qmat_destroy(kv.second);
    g_cache.clear();
    return LOCALAI_OK;
}

#define LQ_LEGACY(NAME, T)                                                                         \
    void localai_##NAME##_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, \
                                 int) {                                                           \
        legacy(T, raw, x, out, rows, cols, 1, false);                                             \
    }                                                                                             \
    void localai_##NAME##_matmul(const uint8_t *raw, const float *v, float *out, int rows, int cols, \
                                 int tokens, int) {                                               \
        legacy(T, raw, v, out, rows, cols, tokens, true);                                         \
    }

LQ_LEGACY(q8_0, LQ_Q8_0)
LQ_LEGACY(q4_0, LQ_Q4_0)
LQ_LEGACY(q4k, LQ_Q4_K)
LQ_LEGACY(q5k, LQ_Q5_K)
LQ_LEGACY(q6k, LQ_Q6_K)

}  // extern "C"
