// The MoE layer with a workspace that lives in the library itself, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that forbid hipMalloc): localai_hip_moe_forward_static.
//
// The workspace is one file-scope device array, `scratch`, of
// LOCALAI_STATIC_WS_BYTES. Each device the library runs on holds its own copy
// until the process ends. Host code never uses the array's name as an
// address: the device address of each device's copy is looked up once, with
// that device current, by hipGetSymbolAddress, and kept per device.
//
// Every call on one device shares that device's array, and each call leaves
// its contents behind. The MoE kernels clear what they need cleared
// themselves (the fused kernel's counter block, the permutation counts), so a
// call does not depend on the previous one's leftovers. Calls that overlap in
// time on one device (different streams or threads) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"

namespace lq {

// 64 MiB: the Qwen3-MoE-style prefill (512 tokens, 128 experts, top-8,
// hidden 2048, intermediate 768) needs 55 MiB; one-token decode of any
// expert count up to 1024 needs a few MiB.
constexpr int64_t STATIC_WS_BYTES = (int64_t)64 << 20;
constexpr int STATIC_WS_MAX_DEVICES = 64;

static __device__ __align__(256) uint8_t scratch[STATIC_WS_BYTES];

static std::mutex g_scratch_mu;
static void *g_scratch_ptr[STATIC_WS_MAX_DEVICES];

// Device address of the current device's `scratch`, looked up on the first
// call for that device.
static int scratch_ptr(void **out) {
    int dev = -1;
    LQ_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= STATIC_WS_MAX_DEVICES) return fail(LOCALAI_ESTATE, "static workspace: device index too large");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(LOCALAI_ESTATE, "static workspace: no device address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return LOCALAI_OK;
}

// Set-up for the current device (called by localai_hip_init).
int static_ws_setup() {
    void *p = nullptr;
    return scratch_ptr(&p);
}

}  // namespace lq

using namespace lq;

extern "C" {

int64_t localai_hip_static_workspace_bytes(void) { return STATIC_WS_BYTES; }

int localai_hip_moe_forward_static(const float *h, int64_t T, int64_t H, const float *rw, const float *rb,
                                   int64_t E, int k, const localai_qmat *gu, const localai_qmat *dn, float *out,
                                   int32_t *topk_idx, float *topk_w, void *stream) {
    clear_error();
    if (!gu || !dn) return fail(LOCALAI_EARG, "moe: null pointer");
    if (T < 1 || H < 1 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E)
        return fail(LOCALAI_EARG, "moe: tokens and hidden >= 1, experts in 1..1024, top_k in 1..min(16, experts)");
    const int64_t need = (int64_t)moe_workspace_bytes(T, E, k, H, gu->g.rows / 2);
    if (need > STATIC_WS_BYTES)
        return fail(LOCALAI_EARG, "moe (static workspace): these sizes need " + std::to_string(need) +
                                      " bytes of workspace, more than the library's " +
                                      std::to_string(STATIC_WS_BYTES));
    // Paths that read the row planes of a handle holding only the tile form
    // (below 32 tokens: Q8_0 rows of partial 256-value blocks, rows over 64
    // blocks of 256, ...) would build them with hipMalloc: refused before
    // any launch.
    if (gu->g.rows % 2 == 0 && moe_would_build_planes(h, T, H, gu, dn))
        return fail(LOCALAI_ETYPE, "moe (static workspace): these experts and sizes take a path that reads row "
                                   "planes the handles do not hold yet; this entry point allocates nothing");
    if (int st = ensure_device()) return st;
    void *ws = nullptr;
    if (int st = scratch_ptr(&ws)) return st;
    NoAllocScope no_alloc;   // qmat_planes refuses rather than allocates, whatever the path
    return localai_hip_moe_forward(h, T, H, rw, rb, E, k, gu, dn, out, topk_idx, topk_w, ws, STATIC_WS_BYTES,
                                   stream);
}

}  // extern "C"
