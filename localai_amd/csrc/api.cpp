// extern "C" entry points: library state, errors, weight handles, dequant, matvec.
#include <hip/hip_runtime.h>

#include <cstring>
#include <atomic>
#include <mutex>
#include <string>

#include "internal.h"

namespace lq {

static thread_local std::string g_error;
static thread_local int g_legacy_status = LOCALAI_OK;
static int g_device = -1;
static std::mutex g_init_mu;

int fail(int status, const std::string &msg) {
    g_error = msg;
    return status;
}

int hip_fail(hipError_t e, const char *what) {
    g_error = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? LOCALAI_ENOMEM : LOCALAI_EHIP;
}

void clear_error() { g_error.clear(); }
void set_legacy_status(int status) { g_legacy_status = status; }

int ensure_device() {
    int dev;
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (g_device < 0) {
            int n = 0;
            hipError_t e = hipGetDeviceCount(&n);
            if (e != hipSuccess || n < 1) return fail(LOCALAI_ESTATE, "no HIP device available");
            const char *env = getenv("LOCALAI_HIP_DEVICE");
            g_device = env ? atoi(env) : 0;
            if (g_device < 0 || g_device >= n) return fail(LOCALAI_ESTATE, "LOCALAI_HIP_DEVICE out of range");
        }
        dev = g_device;
    }
    int cur = -1;
    LQ_HIP(hipGetDevice(&cur));
    if (cur != dev) LQ_HIP(hipSetDevice(dev));
    return LOCALAI_OK;
}

// The MFMA matvec (gemv_mfma.hip) keeps a second, tile-form copy of Q4_K
// weights for single-vector decode; LOCALAI_HIP_MFMA_MATVEC=0 turns it off
// (the row-plane matvec then serves every call).
bool mfma_matvec_enabled() {
    const char *e = getenv("LOCALAI_HIP_MFMA_MATVEC");
    return !(e && e[0] == '0');
}

size_t max_lds_per_block() {
    static std::atomic<int64_t> cached{-1};
    int64_t v = cached.load();
    if (v < 0) {
        int dev = 0, bytes = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            bytes = 64 * 1024;
        v = bytes;
        cached.store(v);
    }
    return (size_t)v;
}

// The row planes of a handle that keeps only the tile form, built once:
// tile form -> GGML bytes (a temporary buffer) -> row planes, on `s`, which
// is then synchronised. Not under graph capture (it allocates and waits).
static std::mutex g_planes_mu;
static thread_local int g_no_alloc = 0;

NoAllocScope::NoAllocScope() { ++g_no_alloc; }
NoAllocScope::~NoAllocScope() { --g_no_alloc; }

const uint8_t *qmat_planes(const localai_qmat *cm, hipStream_t s, int *status) {
    localai_qmat *m = const_cast<localai_qmat *>(cm);
    std::lock_guard<std::mutex> lk(g_planes_mu);
    *status = LOCALAI_OK;
    if (uint8_t *d = __atomic_load_n(&m->data, __ATOMIC_ACQUIRE)) return d;
    if (g_no_alloc) {
        *status = fail(LOCALAI_ETYPE, "this entry point allocates nothing, and the call needs the row planes of a "
                                      "handle that holds only the tile form");
        return nullptr;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        *status = fail(LOCALAI_ESTATE, "qmat: this call needs the row planes, which are built on first use; "
                                       "make the call once outside graph capture first");
        return nullptr;
    }
    uint8_t *planes = nullptr, *ggml = nullptr;
    hipError_t e = hipMalloc(&planes, (size_t)(m->g.matrix_bytes * m->g.batch));
    if (e == hipSuccess) e = hipMalloc(&ggml, (size_t)(m->g.ggml_matrix_bytes * m->g.batch));
    int st = e == hipSuccess ? LOCALAI_OK : hip_fail(e, "hipMalloc(qmat row planes)");
    if (!st) st = launch_mt_unpack(m->g, m->tiles, m->tile_bytes, ggml, s);
    if (!st) st = launch_repack(m->g, ggml, planes, 0, s);
    if (!st) {
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) st = hip_fail(e, "qmat row planes");
    }
    if (ggml) hipFree(ggml);
    if (st) {
        if (planes) hipFree(planes);
        *status = st;
        return nullptr;
    }
    __atomic_store_n(&m->data, planes, __ATOMIC_RELEASE);   // read without the lock elsewhere
    return planes;
}

}  // namespace lq

using namespace lq;

extern "C" {

int localai_hip_version(void) { return 100; }

const char *localai_hip_last_error(void) { return g_error.c_str(); }

int localai_hip_last_status(void) { return g_legacy_status; }

int localai_hip_init(int device) {
    clear_error();
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) return fail(LOCALAI_ESTATE, "no HIP device available");
    if (device < 0 || device >= n) return fail(LOCALAI_EARG, "device index out of range");
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        g_device = device;
    }
    LQ_HIP(hipSetDevice(device));
    // device address of the static workspace (localai_hip_moe_forward_static)
    return static_ws_setup();
}

int localai_hip_block_layout(int t, int *vpb, int *bpb) {
    clear_error();
    if (lq_block_values(t) == 0) return fail(LOCALAI_ETYPE, "unsupported GGML type");
    if (vpb) *vpb = lq_block_values(t);
    if (bpb) *bpb = lq_block_bytes(t);
    return LOCALAI_OK;
}

int localai_hip_dequant(int t, const void *raw, int64_t n, float *out, void *stream) {
    clear_error();
    int bv = lq_block_values(t);
    if (bv == 0) return fail(LOCALAI_ETYPE, "unsupported GGML type");
    if (n < 0 || n % bv) return fail(LOCALAI_EARG, "value count is not a multiple of the block size");
    if (n > 0 && (!raw || !out)) return fail(LOCALAI_EARG, "null pointer");
    if (int st = ensure_device()) return st;
    return launch_dequant_ggml(t, raw, n, out, (hipStream_t)stream);
}

int localai_hip_f32_matvec(const float *w, int64_t rows, int64_t cols, const float *x, int64_t tokens, float *y,
                           void *stream) {
    clear_error();
    if (!w || !x || !y) return fail(LOCALAI_EARG, "null pointer");
    if (rows < 1 || cols < 1 || tokens < 1) return fail(LOCALAI_EARG, "f32 matvec: rows, cols and tokens must be >= 1");
    if (int st = ensure_device()) return st;
    return launch_f32_matvec(w, rows, cols, x, tokens, y, (hipStream_t)stream);
}

int localai_hip_ggml_matvec(int t, const void *w, int64_t rows, int64_t cols, const float *x, int64_t tokens,
                            float *y, void *stream) {
    clear_error();
    if (!w || !x || !y) return fail(LOCALAI_EARG, "null pointer");
    if (int st = ensure_device()) return st;
    return launch_ggml_matvec(t, w, rows, cols, x, tokens, y, (hipStream_t)stream);
}

int localai_hip_zaya_router(const float *r0, const float *b_inp, const float *prev, const float *eda,
                            const float *norm_w, float eps, int64_t r, const float *w_gate, const float *b_gate,
                            int64_t r1, const float *w_mlp2, const float *b_mlp2, int64_t r2, const float *w_mlp4,
                            const float *b_mlp4, int64_t routes, const float *route_bias, float *state,
                            float *probs, int32_t *expert, float *expert_w, void *stream) {
    clear_error();
    if (!r0 || !norm_w || !w_gate || !w_mlp2 || !w_mlp4 || !route_bias || !state || !probs || !expert)
        return fail(LOCALAI_EARG, "null pointer");
    if (r > (1 << 20) || r1 > (1 << 20) || r2 > (1 << 20) || routes > (1 << 20))
        return fail(LOCALAI_EARG, "zaya router: sizes too large");
    if (int st = ensure_device()) return st;
    return launch_zaya_router_tail(r0, b_inp, prev, eda, norm_w, eps, (int)r, w_gate, b_gate, (int)r1, w_mlp2, b_mlp2,
                                   (int)r2, w_mlp4, b_mlp4, (int)routes, route_bias, state, probs, expert,
                                   expert_w, (hipStream_t)stream);
}

int localai_hip_zaya_scale(const float *gu, const float *x, int64_t n, const float *scale, float *y, void *stream) {
    clear_error();
    if (!y) return fail(LOCALAI_EARG, "null pointer");
    if (int st = ensure_device()) return st;
    return launch_zaya_scale(gu, x, n, scale, y, (hipStream_t)stream);
}

int localai_hip_qmat_create(int t, int64_t rows, int64_t cols, int64_t batch, const void *src,
                            int src_is_device, void *stream, localai_qmat **out) {
    clear_error();
    if (!out) return fail(LOCALAI_EARG, "null output handle");
    *out = nullptr;
    if (!lq_repackable(t)) return fail(LOCALAI_ETYPE, "qmat: type must be Q4_0, Q8_0, Q4_K, Q5_K or Q6_K");
    int bv = lq_block_values(t);
    if (rows < 1 || cols < bv || cols % bv || batch < 1)
        return fail(LOCALAI_EARG, "qmat: rows >= 1, batch >= 1 and cols a positive multiple of the block size");
    if (!src) return fail(LOCALAI_EARG, "qmat: null source");
    if (int st = ensure_device()) return st;
    hipStream_t s = (hipStream_t)stream;
    lq_geom g = lq_make_geom(t, rows, cols, batch);
    localai_qmat *m = new localai_qmat;
    m->g = g;
    m->data = nullptr;
    m->tiles = nullptr;
    m->tile_bytes = 0;
    m->row_norm = nullptr;
    hipGetDevice(&m->device);
    // Q4_K / Q6_K / Q8_0 keep only the tile form, which their one-vector
    // matvec, GEMM and MoE kernels read; the row planes are built on first
    // use (qmat_planes). Other types keep the row planes.
    const bool tiled = mfma_matvec_enabled() && mt_matrix_bytes(g) > 0;
    const bool planes_now = !tiled;
    size_t nbytes = (size_t)(g.matrix_bytes * batch);
    hipError_t e = planes_now ? hipMalloc(&m->data, nbytes) : hipSuccess;
    if (e != hipSuccess) { delete m; return hip_fail(e, "hipMalloc(qmat)"); }
    const uint8_t *dsrc = (const uint8_t *)src;
    void *staging = nullptr;
    size_t gbytes = (size_t)(g.ggml_matrix_bytes * batch);
    if (!src_is_device) {
        e = hipMalloc(&staging, gbytes);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, src, gbytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) {
            if (staging) hipFree(staging);
            hipFree(m->data);
            delete m;
            return hip_fail(e, "qmat upload");
        }
        dsrc = (const uint8_t *)staging;
    }
    int st = planes_now ? launch_repack(g, dsrc, m->data, 0, s) : LOCALAI_OK;
    if (st == LOCALAI_OK && tiled) {
        m->tile_bytes = mt_matrix_bytes(g);
        e = hipMalloc(&m->tiles, (size_t)(m->tile_bytes * batch));
        if (e != hipSuccess) {
            m->tiles = nullptr;
            st = hip_fail(e, "hipMalloc(qmat tiles)");
        } else {
            st = launch_mt_repack(g, dsrc, m->tiles, m->tile_bytes, s);
        }
        if (st == LOCALAI_OK) {
            e = hipMalloc(&m->row_norm, (size_t)(2 * batch) * sizeof(float));
            if (e != hipSuccess) {
                m->row_norm = nullptr;
                st = hip_fail(e, "hipMalloc(qmat row norms)");
            } else {
                st = launch_row_norms(g, dsrc, m->row_norm, s);
            }
        }
    }
    if (staging) {
        hipError_t e2 = hipStreamSynchronize(s);
        hipFree(staging);
        if (st == LOCALAI_OK && e2 != hipSuccess) st = hip_fail(e2, "qmat repack");
    }
    if (st != LOCALAI_OK) {
        hipFree(m->data);
        if (m->tiles) hipFree(m->tiles);
        if (m->row_norm) hipFree(m->row_norm);
        delete m;
        return st;
    }
    *out = m;
    return LOCALAI_OK;
}

int localai_hip_qmat_destroy(localai_qmat *m) {
    clear_error();
    if (!m) return LOCALAI_OK;
    if (m->data) hipFree(m->data);
    if (m->tiles) hipFree(m->tiles);
    if (m->row_norm) hipFree(m->row_norm);
    delete m;
    return LOCALAI_OK;
}

int64_t localai_hip_qmat_device_bytes(const localai_qmat *m) {
    if (!m) return 0;
    const uint8_t *planes = __atomic_load_n(&m->data, __ATOMIC_ACQUIRE);
    return (planes ? m->g.matrix_bytes * m->g.batch : 0) + (m->tiles ? m->tile_bytes * m->g.batch : 0);
}

int localai_hip_qmat_unpack(const localai_qmat *m, void *out, void *stream) {
    clear_error();
    if (!m || !out) return fail(LOCALAI_EARG, "null pointer");
    if (int st = ensure_device()) return st;
    const uint8_t *planes = __atomic_load_n(&m->data, __ATOMIC_ACQUIRE);
    if (!planes) return launch_mt_unpack(m->g, m->tiles, m->tile_bytes, (uint8_t *)out, (hipStream_t)stream);
    return launch_repack(m->g, planes, (uint8_t *)out, 1, (hipStream_t)stream);
}

int localai_hip_qmat_dequant(const localai_qmat *m, int64_t expert, float *out, void *stream) {
    clear_error();
    if (!m || !out) return fail(LOCALAI_EARG, "null pointer");
    if (expert < 0 || expert >= m->g.batch) return fail(LOCALAI_EARG, "expert index out of range");
    if (int st = ensure_device()) return st;
    hipStream_t s = (hipStream_t)stream;
    lq_geom one = m->g;
    one.batch = 1;
    void *tmp = nullptr;
    LQ_HIP(hipMalloc(&tmp, (size_t)one.ggml_matrix_bytes));
    const uint8_t *planes = __atomic_load_n(&m->data, __ATOMIC_ACQUIRE);
    int st = planes ? launch_repack(one, planes + expert * m->g.matrix_bytes, (uint8_t *)tmp, 1, s)
                     : launch_mt_unpack(one, m->tiles + expert * m->tile_bytes, m->tile_bytes, (uint8_t *)tmp, s);
    if (st == LOCALAI_OK) st = launch_dequant_ggml(m->g.type, tmp, one.rows * one.cols, out, s);
    hipError_t e = hipStreamSynchronize(s);
    hipFree(tmp);
    if (st == LOCALAI_OK && e != hipSuccess) st = hip_fail(e, "qmat dequant");
    return st;
}

int localai_hip_matvec(const localai_qmat *m, int64_t expert, const float *x, float *y, int ntok,
                       void *stream) {
    clear_error();
    if (!m || !x || !y) return fail(LOCALAI_EARG, "null pointer");
    if (expert < 0 || expert >= m->g.batch) return fail(LOCALAI_EARG, "expert index out of range");
    if (ntok < 1) return fail(LOCALAI_EARG, "ntok must be >= 1");
    if (int st = ensure_device()) return st;
    lq_geom one = m->g;
    one.batch = 1;
    if (m->tiles && ntok == 1 && mt_matvec_ok(one))
        return launch_matvec_mfma(one, m->tiles + expert * m->tile_bytes, x, y, (hipStream_t)stream);
    // several vectors of a tile-form handle: the weights in registers once,
    // each vector through the one-vector arithmetic (no row planes needed)
    if (m->tiles && mt_matvec_ok(one) && (reinterpret_cast<uintptr_t>(x) & 15) == 0)
        return launch_matvec_mfma_tok(one, m->tiles + expert * m->tile_bytes, x, m->g.cols, y, m->g.rows, ntok,
                                      (hipStream_t)stream);
    int st;
    const uint8_t *planes = qmat_planes(m, (hipStream_t)stream, &st);
    if (!planes) return st;
    return launch_matvec(one, planes + expert * m->g.matrix_bytes, x, m->g.cols, y, m->g.rows, ntok,
                         (hipStream_t)stream);
}

int localai_hip_matvec_many(int n, const localai_qmat *const *mats, const int64_t *experts, const float *x,
                            float *const *ys, void *stream) {
    clear_error();
    if (n < 1 || n > 8) return fail(LOCALAI_EARG, "n must be 1..8");
    if (!mats || !x || !ys) return fail(LOCALAI_EARG, "null pointer");
    for (int j = 0; j < n; ++j) {
        if (!mats[j] || !ys[j]) return fail(LOCALAI_EARG, "null pointer");
        const int64_t e = experts ? experts[j] : 0;
        if (e < 0 || e >= mats[j]->g.batch) return fail(LOCALAI_EARG, "expert index out of range");
        if (mats[j]->g.cols != mats[0]->g.cols) return fail(LOCALAI_EARG, "all matrices need the same cols");
    }
    if (int st = ensure_device()) return st;
    hipStream_t s = (hipStream_t)stream;
    // Q4_K / Q6_K matrices with a tile form share one MFMA launch; the rest run one by one
    lq_geom geo[8];
    const lq_geom *gp[8];
    const uint8_t *wt[8];
    float *yp[8];
    int nf = 0;
    for (int j = 0; j < n; ++j) {
        const int64_t e = experts ? experts[j] : 0;
        lq_geom one = mats[j]->g;
        one.batch = 1;
        if (mats[j]->tiles && mt_matvec_ok(one) && one.type == LQ_Q8_0) {
            // Q8_0 on MFMA, a launch of its own
            if (int st = launch_matvec_mfma(one, mats[j]->tiles + e * mats[j]->tile_bytes, x, ys[j], s)) return st;
        } else if (mats[j]->tiles && mt_matvec_ok(one)) {
            geo[nf] = one;
            gp[nf] = &geo[nf];
            wt[nf] = mats[j]->tiles + e * mats[j]->tile_bytes;
            yp[nf] = ys[j];
            ++nf;
        } else {
            int st;
            const uint8_t *planes = qmat_planes(mats[j], s, &st);
            if (!planes) return st;
            if ((st = launch_matvec(one, planes + e * mats[j]->g.matrix_bytes, x, one.cols, ys[j], one.rows, 1, s)))
                return st;
        }
    }
    return nf ? launch_matvec_mfma_many(nf, gp, wt, x, yp, s) : LOCALAI_OK;
}

int64_t localai_hip_matmul_workspace_size(const localai_qmat *m, int64_t tokens) {
    if (!m || tokens < 0) return -1;
    return gemm_workspace_bytes(m->g, tokens);
}

int localai_hip_matmul(const localai_qmat *m, int64_t expert, const float *x, int64_t tokens, float *y,
                       int y_layout, void *ws, int64_t ws_bytes, void *stream) {
    clear_error();
    if (!m || !x || !y) return fail(LOCALAI_EARG, "null pointer");
    if (expert < 0 || expert >= m->g.batch) return fail(LOCALAI_EARG, "expert index out of range");
    if (tokens < 1) return fail(LOCALAI_EARG, "tokens must be >= 1");
    if (y_layout != 0 && y_layout != 1) return fail(LOCALAI_EARG, "y_layout must be 0 or 1");
    if (!ws) return fail(LOCALAI_EARG, "null workspace");
    if (int st = ensure_device()) return st;
    lq_geom one = m->g;
    one.batch = 1;
    const int64_t ts = y_layout == 0 ? m->g.rows : 1, rs = y_layout == 0 ? 1 : tokens;
    // the GEMM reads the tile form where there is one, else the row planes
    return launch_gemm(one, m->tiles ? nullptr : m->data + expert * m->g.matrix_bytes,
                       m->tiles ? m->tiles + expert * m->tile_bytes : nullptr, x, tokens, y, ts, rs, ws, ws_bytes,
                       (hipStream_t)stream);
}

int localai_hip_moe_experts1(const float *h, int64_t H, const localai_qmat *gu, const localai_qmat *dn, int k,
                             const int32_t *expert, const float *weight, int32_t skip, float *out, void *ws,
                             int64_t ws_bytes, void *stream) {
    clear_error();
    if (!h || !gu || !dn || !expert || !weight || !out || !ws) return fail(LOCALAI_EARG, "moe experts: null pointer");
    if (H < 1 || k < 1 || k > 2) return fail(LOCALAI_EARG, "moe experts: hidden >= 1 and top_k 1 or 2");
    const int64_t E = gu->g.batch, I = gu->g.rows / 2;
    if (skip >= 0 && skip < E) return fail(LOCALAI_EARG, "moe experts: skip must be -1 or an index >= experts");
    if (dn->g.batch != E) return fail(LOCALAI_EARG, "moe experts: gate_up and down hold different expert counts");
    if (gu->g.cols != H || gu->g.rows % 2) return fail(LOCALAI_EARG, "moe experts: gate_up must be [E, 2*inter, hidden]");
    if (dn->g.rows != H || dn->g.cols != I) return fail(LOCALAI_EARG, "moe experts: down must be [E, hidden, inter]");
    // shapes the fused kernel does not cover are ETYPE, like unsupported
    // types: the caller falls back to the matvec path
    if (I % 64) return fail(LOCALAI_ETYPE, "moe experts: inter % 64 != 0");
    if (ws_bytes < (int64_t)moe_workspace_bytes(1, E, k, H, I)) return fail(LOCALAI_EARG, "moe experts: workspace too small");
    if ((reinterpret_cast<uintptr_t>(h) & 15) || (reinterpret_cast<uintptr_t>(ws) & 255))
        return fail(LOCALAI_EARG, "moe experts: h must be 16-byte and workspace 256-byte aligned");
    if (int st = ensure_device()) return st;
    return launch_moe_experts1(h, H, gu, dn, k, expert, weight, skip, out, ws, (hipStream_t)stream);
}

int localai_hip_moe_error(const void *ws, int64_t T, int64_t E, void *stream) {
    clear_error();
    if (!ws || T < 1 || E < 1) return fail(LOCALAI_EARG, "moe error: null workspace or sizes < 1");
    if (int st = ensure_device()) return st;
    uint32_t word = 0;
    if (int st = moe_error_word(ws, T, E, (hipStream_t)stream, &word)) return st;
    if (word & 2u) return fail(LOCALAI_EARG, "moe: an expert index was outside [0, experts) and not the skip route");
    if (word & 1u) return fail(LOCALAI_EHIP, "moe: a wait of the fused expert kernel ran out (output rows are NaN)");
    return LOCALAI_OK;
}

int localai_hip_debug_fused_wait(int spin_limit, int producers_count) {
    clear_error();
    set_layer_wait(spin_limit, producers_count);
    return set_fused_wait(spin_limit, producers_count);
}

int localai_hip_stream_read(const void *src, int64_t bytes, uint32_t *out, void *stream) {
    clear_error();
    if (!src || !out) return fail(LOCALAI_EARG, "stream read: null pointer");
    if (bytes < 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15))
        return fail(LOCALAI_EARG, "stream read: bytes a multiple of 16 and a 16-byte aligned source");
    if (int st = ensure_device()) return st;
    return launch_stream_read(src, bytes, out, (hipStream_t)stream);
}

int64_t localai_hip_layer_workspace_size(int64_t dim, int64_t ffn) {
    if (dim < 1 || ffn < 1) return -1;
    return (int64_t)layer_workspace_bytes(dim, ffn);
}

int localai_hip_layer_chain(const localai_qmat *const *mats, const float *pre, const float *att,
                            const float *w_ffn, const float *w_attn, float eps, const float *rope_cos,
                            const float *rope_sin, int head_dim, int rope_half, float *x_out, float *q_out,
                            float *k_out, float *v_out, void *ws, int64_t ws_bytes, void *stream) {
    clear_error();
    if (!mats || !pre || !att || !w_ffn || !w_attn || !x_out || !q_out || !k_out || !v_out || !ws)
        return fail(LOCALAI_EARG, "layer chain: null pointer");
    for (int i = 0; i < 7; ++i) {
        const localai_qmat *m = mats[i];
        if (!m) return fail(LOCALAI_EARG, "layer chain: null matrix handle");
        if (m->g.batch != 1) return fail(LOCALAI_EARG, "layer chain: matrices must be plain 2-D tensors");
        if ((m->g.type != LQ_Q4_K && m->g.type != LQ_Q6_K) || !m->tiles)
            return fail(LOCALAI_ETYPE, "layer chain: Q4_K / Q6_K matrices with the tile form only");
    }
    const int64_t dim = mats[0]->g.rows, ffn = mats[1]->g.rows;
    if (mats[0]->g.cols != dim) return fail(LOCALAI_EARG, "layer chain: attn_output must be [dim, dim]");
    if (dim % 256 || ffn % 256) return fail(LOCALAI_ETYPE, "layer chain: dim and ffn must be multiples of 256");
    if (mats[1]->g.cols != dim || mats[2]->g.rows != ffn || mats[2]->g.cols != dim ||
        mats[2]->g.type != mats[1]->g.type)
        return fail(LOCALAI_EARG, "layer chain: ffn_gate and ffn_up must be [ffn, dim] of one type");
    if (mats[3]->g.rows != dim || mats[3]->g.cols != ffn) return fail(LOCALAI_EARG, "layer chain: ffn_down must be [dim, ffn]");
    for (int i = 4; i < 7; ++i)
        if (mats[i]->g.cols != dim) return fail(LOCALAI_EARG, "layer chain: attn_q / attn_k / attn_v must have dim columns");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(LOCALAI_EARG, "layer chain: rope_cos and rope_sin go together");
    if (rope_cos && (head_dim < 2 || head_dim % 2 || rope_half < 0 || 2 * rope_half > head_dim))
        return fail(LOCALAI_EARG, "layer chain: RoPE needs an even head_dim and rope_half <= head_dim / 2");
    if (ws_bytes < (int64_t)layer_workspace_bytes(dim, ffn)) return fail(LOCALAI_EARG, "layer chain: workspace too small");
    auto mis = [](const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & m) != 0; };
    if (mis(pre, 15) || mis(att, 15) || mis(x_out, 15) || mis(w_ffn, 15) || mis(w_attn, 15) || mis(ws, 255))
        return fail(LOCALAI_EARG, "layer chain: pre, att, x_out and the norm weights 16-byte, workspace 256-byte aligned");
    if (int st = ensure_device()) return st;
    return launch_layer_chain(mats, pre, att, w_ffn, w_attn, eps, rope_cos, rope_sin, head_dim, rope_half, x_out,
                              q_out, k_out, v_out, ws, (hipStream_t)stream);
}

int localai_hip_layer_chain_mode(int one_launch) {
    clear_error();
    return set_layer_mode(one_launch);
}

int localai_hip_layer_error(void *ws, void *stream) {
    clear_error();
    if (!ws) return fail(LOCALAI_EARG, "layer error: null workspace");
    if (int st = ensure_device()) return st;
    uint32_t word = 0;
    if (int st = layer_error_word(ws, (hipStream_t)stream, &word)) return st;
    if (word) return fail(LOCALAI_EHIP, "layer chain: a wait between stages ran out (outputs are NaN)");
    return LOCALAI_OK;
}

int64_t localai_hip_attention_workspace_size(int64_t max_seq, int n_heads, int n_kv, int head_dim) {
    if (max_seq < 1 || n_heads < 1 || n_kv < 1 || n_heads % n_kv || head_dim < 1) return -1;
    return (int64_t)attention_workspace_bytes(max_seq, n_heads, n_kv, head_dim);
}

int localai_hip_attention_decode(const float *q, const float *k_new, const float *v_new, float *kc, float *vc,
                                 int64_t position, int64_t max_seq, int n_heads, int n_kv, int head_dim,
                                 int64_t window, const float *gate, float *out, void *ws, int64_t ws_bytes,
                                 void *stream) {
    clear_error();
    if (!q || !kc || !vc || !out) return fail(LOCALAI_EARG, "attention: null pointer");
    if ((k_new == nullptr) != (v_new == nullptr)) return fail(LOCALAI_EARG, "attention: k_new and v_new go together");
    if (n_heads < 1 || n_kv < 1 || n_heads % n_kv)
        return fail(LOCALAI_EARG, "attention: n_heads must be a positive multiple of n_kv_heads");
    if (head_dim < 1) return fail(LOCALAI_EARG, "attention: head_dim must be >= 1");
    if (max_seq < 1 || position < 0 || position >= max_seq)
        return fail(LOCALAI_EARG, "attention: position must be in [0, max_seq)");
    if (window < 0) return fail(LOCALAI_EARG, "attention: window must be >= 0");
    auto mis = [](const void *p) { return p && (reinterpret_cast<uintptr_t>(p) & 15) != 0; };
    if (mis(q) || mis(k_new) || mis(v_new) || mis(kc) || mis(vc) || mis(gate) || mis(out) || mis(ws))
        return fail(LOCALAI_EARG, "attention: every buffer must be 16-byte aligned");
    if (int st = ensure_device()) return st;
    return launch_attention_decode(q, k_new, v_new, kc, vc, position, window, n_heads, n_kv, head_dim, gate, out,
                                   ws, ws_bytes, (hipStream_t)stream);
}

int localai_hip_delta_net_step(float *state, const float *q, const float *k, const float *v, const float *decay,
                               const float *beta, float *core, int heads, int key_dim, int value_dim,
                               void *stream) {
    clear_error();
    if (!state || !q || !k || !v || !decay || !beta || !core) return fail(LOCALAI_EARG, "delta net: null pointer");
    if (heads < 1 || key_dim < 1 || value_dim < 1 || heads > 65535)
        return fail(LOCALAI_EARG, "delta net: heads in 1..65535, key_dim and value_dim >= 1");
    if ((int64_t)heads * key_dim * value_dim > ((int64_t)1 << 40)) return fail(LOCALAI_EARG, "delta net: state too large");
    if (int st = ensure_device()) return st;
    return launch_delta_net(state, q, k, v, decay, beta, core, heads, key_dim, value_dim, (hipStream_t)stream);
}

int64_t localai_hip_moe_workspace_size(int64_t T, int64_t E, int k, int64_t H, int64_t I) {
    if (T < 1 || E < 1 || k < 1 || H < 1 || I < 1) return -1;
    return (int64_t)moe_workspace_bytes(T, E, k, H, I);
}

int localai_hip_moe_table_offsets(int64_t T, int64_t E, int k, int64_t H, int64_t I, int64_t *offs) {
    clear_error();
    if (T < 1 || E < 1 || k < 1 || H < 1 || I < 1 || !offs)
        return fail(LOCALAI_EARG, "moe table offsets: sizes must be >= 1 and offs not null");
    const MoeLayout L = moe_layout(T, E, k, H, I);
    const int64_t v[12] = {L.counts, L.offsets, L.active, L.n_active, L.perm,  L.pos,
                           L.tile_e, L.tile_p0, L.tile_n, L.n_tiles, L.max_tiles, L.max_tiles > 0 ? moe_gemm_tile() : 0};
    for (int i = 0; i < 12; ++i) offs[i] = v[i];
    return LOCALAI_OK;
}

int localai_hip_moe_expert_gemm(const localai_qmat *gu, const localai_qmat *dn, int64_t T, int64_t E, int k,
                                void *ws, int64_t ws_bytes, int which, void *stream) {
    clear_error();
    if (!gu || !dn || !ws) return fail(LOCALAI_EARG, "moe expert gemm: null pointer");
    if (which != 0 && which != 1) return fail(LOCALAI_EARG, "moe expert gemm: which is 0 (gate_up) or 1 (down)");
    if (T < 1 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E || gu->g.batch != E || dn->g.batch != E ||
        gu->g.rows % 2 || dn->g.rows != gu->g.cols || dn->g.cols != gu->g.rows / 2)
        return fail(LOCALAI_EARG, "moe expert gemm: sizes as for localai_hip_moe_forward");
    if (ws_bytes < (int64_t)moe_workspace_bytes(T, E, k, gu->g.cols, gu->g.rows / 2) ||
        (reinterpret_cast<uintptr_t>(ws) & 255))
        return fail(LOCALAI_EARG, "moe expert gemm: workspace too small or not 256-byte aligned");
    if (int st = ensure_device()) return st;
    return launch_moe_expert_gemm(gu, dn, T, E, k, ws, which, (hipStream_t)stream);
}

int localai_hip_moe_forward(const float *h, int64_t T, int64_t H, const float *rw, const float *rb,
                            int64_t E, int k, const localai_qmat *gu, const localai_qmat *dn, float *out,
                            int32_t *topk_idx, float *topk_w, void *ws, int64_t ws_bytes, void *stream) {
    clear_error();
    if (!h || !rw || !gu || !dn || !out || !topk_idx || !topk_w || !ws) return fail(LOCALAI_EARG, "moe: null pointer");
    if (T < 1 || H < 1) return fail(LOCALAI_EARG, "moe: tokens and hidden must be >= 1");
    if (E < 1 || E > 1024) return fail(LOCALAI_EARG, "moe: experts must be in 1..1024");
    if (k < 1 || k > 16 || k > E) return fail(LOCALAI_EARG, "moe: top_k must be in 1..min(16, experts)");
    const int64_t I = gu->g.rows / 2;
    if (gu->g.batch != E || dn->g.batch != E) return fail(LOCALAI_EARG, "moe: expert tensors must hold `experts` matrices");
    if (gu->g.cols != H || gu->g.rows % 2 || I % 64) return fail(LOCALAI_EARG, "moe: gate_up must be [E, 2*inter, hidden] with inter % 64 == 0");
    if (dn->g.rows != H || dn->g.cols != I) return fail(LOCALAI_EARG, "moe: down must be [E, hidden, inter]");
    if (ws_bytes < (int64_t)moe_workspace_bytes(T, E, k, H, I)) return fail(LOCALAI_EARG, "moe: workspace too small");
    if ((reinterpret_cast<uintptr_t>(h) & 15) || (reinterpret_cast<uintptr_t>(rw) & 15) ||
        (reinterpret_cast<uintptr_t>(ws) & 255))
        return fail(LOCALAI_EARG, "moe: h and router_w must be 16-byte and workspace 256-byte aligned");
    if (int st = ensure_device()) return st;
    return launch_moe(h, T, H, rw, rb, E, k, gu, dn, out, topk_idx, topk_w, ws, (hipStream_t)stream);
}

}  // extern "C"
