// Internal interfaces shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "qformat.h"
#include "../../include/localai_hip.h"

struct localai_qmat {
    lq_geom g;
    uint8_t *data;      // device, g.matrix_bytes * g.batch (row planes, qformat.h); for types with a
                        // tile form null until qmat_planes builds it
    int device;
    uint8_t *tiles;     // device, MFMA tile form (gemv_mfma.hip) or null
    int64_t tile_bytes; // per matrix of the tile form
    float *row_norm;    // device, with the tile form: per matrix, the largest row L2 norm of rows
                        // [0, rows / 2) and of rows [rows / 2, rows) (gate_up: gate and up), rounded up
};

namespace lq {

// Error state (thread-local), set by the entry points.
int fail(int status, const std::string &msg);
int hip_fail(hipError_t e, const char *what);
void clear_error();
void set_legacy_status(int status);

#define LQ_HIP(expr)                                      \
    do {                                                  \
        hipError_t _e = (expr);                           \
        if (_e != hipSuccess) return lq::hip_fail(_e, #expr); \
    } while (0)

int ensure_device();   // make the library's device current for this thread
int static_ws_setup(); // look up the current device's static workspace (static_ws.hip)
size_t max_lds_per_block();   // LDS bytes a workgroup may use on the current device

// launchers (return LOCALAI_* status)
int launch_repack(const lq_geom &g, const uint8_t *ggml, uint8_t *packed, int direction,
                  hipStream_t s);
int launch_dequant_ggml(int t, const void *raw, int64_t n, float *out, hipStream_t s);
int launch_f32_matvec(const float *W, int64_t rows, int64_t cols, const float *x, int64_t ntok, float *y,
                      hipStream_t s);
// matvec from GGML bytes on the device (F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0; ggml_matvec.hip)
int launch_ggml_matvec(int t, const void *W, int64_t rows, int64_t cols, const float *x, int64_t ntok, float *y,
                       hipStream_t s);
struct GemvPlan {
    int waves;        // waves per workgroup (split the K units)
    int slots;        // 64-value units per lane per wave
    int rows;         // rows per workgroup
    int lpr;          // lanes per row (64, or 32 / 16 for short rows)
    size_t lds_bytes; // dynamic LDS (x staging) per workgroup
};
GemvPlan gemv_plan(const lq_geom &g, int nt);
int launch_matvec(const lq_geom &g, const uint8_t *packed, const float *x, int64_t x_stride,
                  float *y, int64_t y_stride, int ntok, hipStream_t s);

int64_t mt_matrix_bytes(const lq_geom &g);
int launch_mt_repack(const lq_geom &g, const uint8_t *ggml, uint8_t *dst, int64_t dst_matrix_bytes, hipStream_t s);
// largest row L2 norms of the two row halves of every matrix of GGML bytes
// (localai_qmat::row_norm; out: 2 * batch floats, cleared here)
int launch_row_norms(const lq_geom &g, const uint8_t *ggml, float *out, hipStream_t s);
// tile form -> GGML bytes (the inverse of launch_mt_repack)
int launch_mt_unpack(const lq_geom &g, const uint8_t *tiles, int64_t tile_matrix_bytes, uint8_t *ggml,
                     hipStream_t s);
// The row planes of a handle (built from the tile form on first use, then
// kept; not under graph capture); null with *status set on failure
const uint8_t *qmat_planes(const localai_qmat *m, hipStream_t s, int *status);
bool mt_matvec_ok(const lq_geom &g);
int launch_matvec_mfma(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, hipStream_t s);
// several vectors x[t] (stride ldx) through the one-vector MFMA arithmetic, weights read once
int launch_matvec_mfma_tok(const lq_geom &g, const uint8_t *Wt, const float *x, int64_t ldx, float *y, int64_t ldy,
                           int ntok, hipStream_t s);
int launch_matvec_mfma_many(int n, const lq_geom *const *g, const uint8_t *const *Wt, const float *x,
                            float *const *y, hipStream_t s);
// the decode step's glue around a matvec (gemv_mfma.hip): prologue PRO / epilogue EPI
enum { MT_PRO_X = 0, MT_PRO_NORM = 1 };
enum { MT_EPI_Y = 0, MT_EPI_RES = 1, MT_EPI_ROPE = 2, MT_EPI_SILU = 3, MT_EPI_PAIR = 4 };
constexpr int MT_SSQ = 512;   // floats of a per-tile sums-of-squares buffer
struct MtGlue {
    const float *ssq_in;       // NORM: sums of squares of src over its 16-value tiles [MT_SSQ], zero past n / 16
    int n;                     // NORM: values of src (at most 8192)
    float eps;
    const float *res;          // RES: residual [rows]
    float *ssq_out;            // RES: sums of y^2 over each 16-row tile, or null
    const float *w_next;       // RES: y_next = y * w_next (the next norm's weight), or null
    float *y_next;
    const float *cos, *sin;    // ROPE: [rope_half]
    int head_dim, rope_half, rope_jobs;
    const uint8_t *Wt2;        // SILU, PAIR: the second matrix (tile form; up, W being the gate)
    float *y2;                 // PAIR: its output
};
// one matrix: (X, RES) or (NORM, SILU) over paired gate / up tiles; fused
// matrices sharing x: (NORM, Y) or (NORM, ROPE)
int launch_matvec_mfma_glue(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, int pro, int epi,
                            const MtGlue &gl, hipStream_t s);
int launch_matvec_mfma_many_glue(int n, const lq_geom *const *g, const uint8_t *const *Wt, const float *x,
                                 float *const *y, int pro, int epi, const MtGlue &gl, hipStream_t s);
bool mfma_matvec_enabled();

int64_t gemm_workspace_bytes(const lq_geom &g, int64_t ntok);
// Wt: the tile form (mfma_core.h) when the handle has one, else null
int launch_gemm(const lq_geom &g, const uint8_t *packed, const uint8_t *Wt, const float *x, int64_t ntok, float *y,
                int64_t y_ts, int64_t y_rs, void *ws, int64_t ws_bytes, hipStream_t s);

// nrm2 (not null, row layout only): each row's sum of squares
int launch_x_to_f16(const float *X, int64_t ldx, int64_t cols, const int32_t *rows_map, int k, int64_t ntok,
                    _Float16 *Xh, int64_t ldh, float *inv, hipStream_t s, int tiled = 0, float *nrm2 = nullptr);
// The gate_up expert GEMM's f16 output (GemmArgs::Yh): the down GEMM's input
// rows and their scales written directly.
struct MoeF16Out {
    _Float16 *Yh;
    int64_t ldy;
    float *inv_out;
    const float *wnorm, *xnorm2;
};
int launch_moe_gemm(const lq_geom &g, const uint8_t *Wall, const uint8_t *Wt_all, int64_t wt_bytes, bool gate_up,
                    const _Float16 *Xh, int64_t ldh, const float *inv, const int32_t *rows_map, int rows_k,
                    float *Y, int64_t y_ts, int64_t inter, const int32_t *tile_e, const int32_t *tile_p0,
                    const int32_t *tile_n, const int32_t *n_tiles, int max_tiles, hipStream_t s,
                    const MoeF16Out *f16_out = nullptr);
int moe_gemm_tile();   // tokens per expert GEMM tile

int launch_zaya_router_tail(const float *r0, const float *b0, const float *prev, const float *eda,
                            const float *norm_w, float eps, int R, const float *W1, const float *b1, int R1,
                            const float *W2, const float *b2, int R2, const float *W3, const float *b3, int NE,
                            const float *bias, float *state, float *probs, int32_t *expert, float *expert_w,
                            hipStream_t s);
int launch_zaya_scale(const float *gu, const float *x, int64_t n, const float *scale, float *y, hipStream_t s);

struct MoeLayout {
    int64_t logits, sync, counts, offsets, active, n_active, perm, pos, act, ysl;
    int64_t tile_e, tile_p0, tile_n, n_tiles, xh_gu, inv_gu, hn2, xh_dn, inv_dn;
    int64_t max_tiles, bytes;
};
MoeLayout moe_layout(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I);
size_t moe_workspace_bytes(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I);
// one expert GEMM of the prefill path again, on the tables the last launch_moe left in ws
int launch_moe_expert_gemm(const localai_qmat *gu, const localai_qmat *dn, int64_t T, int64_t E, int k, void *ws,
                           int which, hipStream_t s);
// true when launch_moe would build a handle's row planes (allocate) for these sizes
bool moe_would_build_planes(const float *h, int64_t T, int64_t H, const localai_qmat *gu, const localai_qmat *dn);
// While set on a thread, qmat_planes refuses to build planes (LOCALAI_ETYPE)
// instead of allocating: the no-allocation entry points set it around their work.
struct NoAllocScope {
    NoAllocScope();
    ~NoAllocScope();
};
int launch_moe(const float *h, int64_t T, int64_t H, const float *rw, const float *rb, int64_t E, int k,
               const localai_qmat *gu, const localai_qmat *dn, float *out, int32_t *topk_idx, float *topk_w,
               void *ws, hipStream_t s);
// error word of the fused one-token expert kernel in a MoE workspace (after
// the stream has finished); test controls of its waits
int moe_error_word(const void *ws, int64_t T, int64_t E, hipStream_t s, uint32_t *word);
int set_fused_wait(int spin, int count);
int launch_stream_read(const void *src, int64_t bytes, uint32_t *out, hipStream_t s);

// decode-layer matvec chain (layer.hip); m: o, gate, up, down, q, k, v
size_t layer_workspace_bytes(int64_t dim, int64_t ffn);
int launch_layer_chain(const localai_qmat *const *m, const float *pre, const float *att, const float *w_ffn,
                       const float *w_attn, float eps, const float *rope_cos, const float *rope_sin, int head_dim,
                       int rope_half, float *x_out, float *q_out, float *k_out, float *v_out, void *ws,
                       hipStream_t s);
int layer_error_word(void *ws, hipStream_t s, uint32_t *word);
int set_layer_wait(int spin, int count);
int set_layer_mode(int one_launch);
int launch_moe_experts1(const float *h, int64_t H, const localai_qmat *gu, const localai_qmat *dn, int k,
                        const int32_t *topk_idx, const float *topk_w, int skip, float *out, void *ws,
                        hipStream_t s);

// decode-step attention mixers (attention.hip)
size_t attention_workspace_bytes(int64_t max_seq, int n_heads, int n_kv, int hd);
int launch_attention_decode(const float *q, const float *k_new, const float *v_new, float *kc, float *vc,
                            int64_t position, int64_t window, int n_heads, int n_kv, int hd, const float *gate,
                            float *out, void *ws, int64_t ws_bytes, hipStream_t s);
int launch_delta_net(float *state, const float *q, const float *k, const float *v, const float *decay,
                     const float *beta, float *core, int heads, int KD, int VD, hipStream_t s);

}  // namespace lq
