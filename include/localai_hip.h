/*
 * localai_hip.h -- C ABI of liblocalai_hip.so, the MI355X (gfx950) quantized
 * matvec / GEMM / MoE library.
 *
 * Two groups of entry points:
 *
 *  1. The reference's ten legacy exports, same names, argument order and
 *     meaning as engine/native_quant.cpp:705-768 (bound by ctypes in
 *     engine/native_quant.py:77-94). Host pointers in, host results out; the
 *     work runs on the GPU. `threads` is accepted and ignored.
 *
 *  2. Device-pointer entry points (prefix localai_hip_). Every pointer named
 *     *_dev is a device address, `stream` is a hipStream_t (NULL = the legacy
 *     default stream). They return 0 on success or a LOCALAI_E* status; the
 *     message of the last failure on the calling thread is available from
 *     localai_hip_last_error(). Nothing throws across this boundary.
 *
 * Weights live on the device in a repacked, lane-interleaved form held by an
 * opaque localai_qmat handle, created from GGML bytes (host or device).
 */
#ifndef LOCALAI_HIP_H
#define LOCALAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LOCALAI_OK 0
#define LOCALAI_EARG 1      /* bad argument (size, shape, null pointer) */
#define LOCALAI_ETYPE 2     /* GGML type not supported by this entry point */
#define LOCALAI_EHIP 3      /* HIP runtime error */
#define LOCALAI_ENOMEM 4    /* device allocation failed */
#define LOCALAI_ESTATE 5    /* library not initialised / no device */

typedef struct localai_qmat localai_qmat;

/* ---- library state ------------------------------------------------------ */

/* ABI version (major*100 + minor). */
int localai_hip_version(void);

/* Select the HIP device used by this thread's calls; idempotent. */
int localai_hip_init(int device);

/* Message of the last failing call on this thread ("" if none). */
const char *localai_hip_last_error(void);

/* Status of the last legacy (void-returning) call on this thread. */
int localai_hip_last_status(void);

/* (values per block, bytes per block) of a GGML type; engine/dequant.py:12-17.
 * Returns LOCALAI_ETYPE for types engine/dequant.py rejects. */
int localai_hip_block_layout(int ggml_type, int *values_per_block, int *bytes_per_block);

/* ---- dequantisation (engine/dequant.py:27-167) -------------------------- */

/* Decode n_values of GGML type `ggml_type` from raw_dev (GGML bytes) to fp32.
 * All ten engine/dequant.py types. Bit-exact with the reference decoders. */
int localai_hip_dequant(int ggml_type, const void *raw_dev, int64_t n_values,
                        float *out_dev, void *stream);

/* y[t, r] = sum_c w[r, c] * x[t, c] for an fp32 matrix w [rows, cols] and
 * x [tokens, cols] -> y [tokens, rows] (all device, row-major): the device
 * path for F32 GGUF matrices (and any matrix already decoded to fp32 by
 * localai_hip_dequant); it replaces the reference's NumPy `weights @ x`
 * (engine/gguf_parser.py:269-289, :350-358). Results do not depend on the
 * launch (fixed summation order). */
int localai_hip_f32_matvec(const float *w_dev, int64_t rows, int64_t cols, const float *x_dev,
                           int64_t tokens, float *y_dev, void *stream);

/* y[t, r] = sum_c W[r, c] * x[t, c] for t < tokens, straight from the GGML
 * bytes of W [rows, cols] on the device (the file's bytes, no expansion):
 * F16, Q4_1, Q5_0, Q5_1 -- the types without a packed kernel -- and F32,
 * Q4_0, Q8_0. Each block is decoded in registers with the formulas of
 * engine/dequant.py (bit-identical values) and multiplied in fp32 with a
 * fixed summation order. Replaces the dequantize + NumPy `weights @ x`
 * fallback of GGUFFile.matvec / .matmul (engine/gguf_parser.py:269-289,
 * :350-358) and its fp32 / fp16 matrix caches (:65-69). cols a multiple of 8
 * and of the block size; x 16-byte aligned (and W for F32 / F16); y is
 * [tokens, rows]. LOCALAI_ETYPE for other types. */
int localai_hip_ggml_matvec(int ggml_type, const void *w_dev, int64_t rows, int64_t cols, const float *x_dev,
                            int64_t tokens, float *y_dev, void *stream);

/* ---- device-resident weight matrices ------------------------------------ */

/* Upload + repack a [batch, rows, cols] GGML tensor (batch = 1 for a plain
 * matrix, = experts for a 3-D expert tensor, engine/zaya.py:139-150).
 * `src_is_device` says whether ggml_bytes is a device address. Types:
 * Q4_0, Q8_0, Q4_K, Q5_K, Q6_K (the reference's native types,
 * engine/native_quant.py:104). cols must be a multiple of the block size.
 * Q4_K, Q6_K and Q8_0 handles hold the MFMA tile form only (the same bytes
 * as GGML, reordered); the row-plane form that the several-vector matvec,
 * the Q8_0 matvec of rows that are not whole 256-value super-blocks and the
 * fallback MoE paths read is built from it on the first such call (which
 * allocates and waits for the stream, so not under graph capture:
 * LOCALAI_ESTATE there) and then kept. Other types hold the row planes.
 * With the tile form a handle also keeps, per matrix, the largest row L2
 * norm of its first and of its second half of rows (8 bytes per matrix;
 * the prefill MoE gate_up GEMM scales its f16 outputs from them). */
int localai_hip_qmat_create(int ggml_type, int64_t rows, int64_t cols, int64_t batch,
                            const void *ggml_bytes, int src_is_device, void *stream,
                            localai_qmat **out);
int localai_hip_qmat_destroy(localai_qmat *m);

/* Device bytes held by the handle (tile form, and row planes once built). */
int64_t localai_hip_qmat_device_bytes(const localai_qmat *m);

/* Write the GGML bytes back out (inverse of the repack) to out_dev. */
int localai_hip_qmat_unpack(const localai_qmat *m, void *out_dev, void *stream);

/* Dequantise expert `expert` of a handle to fp32 [rows, cols]. */
int localai_hip_qmat_dequant(const localai_qmat *m, int64_t expert, float *out_dev,
                             void *stream);

/* y[t, r] = sum_c W_e[r, c] * x[t, c] for t < ntok (decode matvec).
 * x_dev is [ntok, cols] fp32 row-major, y_dev is [ntok, rows] fp32.
 * One vector (ntok = 1) of a Q4_K, Q6_K or Q8_0 handle whose rows are whole
 * 256-value super-blocks: int8 MFMA over the raw quants, x split exactly
 * into three int8 pieces per scale group (21 bits of each value against the
 * group maximum), the integer dot products exact, recombined and scaled in
 * fp32 (normwise error about 1e-6); from 2048 row tiles one workgroup per CU
 * loops over the tiles (same arithmetic, same bits). 2..31 vectors of such
 * a handle: the same arithmetic per vector over the tile form, the weights
 * read once per call (each y[t] equal to the one-vector call on x[t]). Other
 * types: fp32 products of exactly decoded weights, fp32 accumulation (the
 * vectors two per launch while cols <= 8192, one otherwise). */
int localai_hip_matvec(const localai_qmat *m, int64_t expert, const float *x_dev,
                       float *y_dev, int ntok, void *stream);

/* Several decode matvecs that share one input vector:
 *   ys_dev[j][r] = sum_c W_j[r, c] * x[c],  W_j = matrix experts[j] of mats[j]
 * (experts may be NULL: matrix 0 of every handle). Counterpart of consecutive
 * mat() calls on one vector -- attn_q/k/v (engine/model.py:185-187) and
 * ffn_gate/up (engine/model.py:232) -- with the Q4_K / Q6_K matrices computed
 * in one launch (results identical to localai_hip_matvec on each matrix).
 * 1 <= n <= 8; every matrix must have the same cols. */
int localai_hip_matvec_many(int n, const localai_qmat *const *mats, const int64_t *experts,
                            const float *x_dev, float *const *ys_dev, void *stream);

/* ---- prefill matmul (MFMA) ---------------------------------------------- */

/* Bytes of device workspace localai_hip_matmul needs for `tokens` rows of x. */
int64_t localai_hip_matmul_workspace_size(const localai_qmat *m, int64_t tokens);

/* Many-token product with matrix `expert` of the handle; counterpart of
 * localai_*_matmul (engine/native_quant.cpp:744-768, decoded_matmul_row
 * :444-531), whose output is [rows, tokens]:
 *   x_dev  [tokens, cols] fp32 row-major
 *   y_dev  y_layout 0: [tokens, rows] (x @ W^T);  1: [rows, tokens]
 * Weights are decoded exactly in fp32 and rounded once to f16; each token row
 * of x is scaled by a power of two into f16 range and rounded to f16; MFMA
 * f16 products with fp32 accumulation (normwise error about 2^-12). */
int localai_hip_matmul(const localai_qmat *m, int64_t expert, const float *x_dev, int64_t tokens,
                       float *y_dev, int y_layout, void *workspace_dev, int64_t workspace_bytes,
                       void *stream);

/* ---- decode layer: the matvec chain in one launch ----------------------- */

/* Bytes of workspace localai_hip_layer_chain needs. The workspace must be
 * zero-filled before its first use; every launch leaves it so. */
int64_t localai_hip_layer_workspace_size(int64_t dim, int64_t ffn);

/* The matvecs of one decode layer with the glue between them, from the
 * attention output of layer L to the attention inputs of layer L+1
 * (engine/model.py:229-233 of layer L, then :182-185 and :203-213 of L+1):
 *   x1 = pre + W_o att
 *   act = silu(W_gate u) * (W_up u),   u = norm(x1) * w_ffn
 *   x_out = x1 + W_down act
 *   q, k, v = W_q v', W_k v', W_v v',   v' = norm(x_out) * w_attn
 * norm(x) = x / sqrt(mean(x^2) + eps) (engine/model.py:82, the mean in fp64);
 * silu as engine/model.py:232. With rope_cos / rope_sin ([rope_half] each,
 * cos / sin of position * inv_freq as the caller computes them,
 * engine/model.py:190-203) q and k get Llama's adjacent-pair RoPE in every
 * head of head_dim values (:205-210); NULL for none.
 * mats: the seven handles in the order attn_output, ffn_gate, ffn_up,
 * ffn_down, attn_q, attn_k, attn_v of layer L+1 (w_attn is its attn_norm),
 * each a Q4_K or Q6_K matrix with the tile form; dim and ffn multiples of
 * 256; w_ffn / w_attn 16-byte aligned. By default the chain runs as four
 * launches on `stream` (o; gate + up; down; q + k + v) with the norms,
 * SiLU*up, the residual adds and RoPE fused into the matvec kernels'
 * prologues and epilogues (dim at most 8192, ffn at most 18432; larger
 * layers run as one launch). localai_hip_layer_chain_mode(1) selects one
 * launch always, whose stages' workgroups run in stage order and
 * each wait on the device for the stage before it after requesting their
 * own weights. Matvec arithmetic is that of localai_hip_matvec. ETYPE for
 * shapes or types without a kernel (the caller then runs the separate
 * matvecs). Calls on one workspace must not overlap. */
int localai_hip_layer_chain(const localai_qmat *const *mats, const float *pre_dev, const float *att_dev,
                            const float *w_ffn_dev, const float *w_attn_dev, float eps,
                            const float *rope_cos_dev, const float *rope_sin_dev, int head_dim,
                            int rope_half, float *x_out_dev, float *q_dev, float *k_dev, float *v_dev,
                            void *workspace_dev, int64_t workspace_bytes, void *stream);

/* Process-wide choice of how localai_hip_layer_chain runs: 0 (the default)
 * four launches with the glue fused into the matvecs, 1 one launch with
 * device-side waits between the stages. No counterpart in the reference. */
int localai_hip_layer_chain_mode(int one_launch);

/* Waits for `stream`, then reports whether a wait between the stages of the
 * last localai_hip_layer_chain launches on this workspace ran out
 * (LOCALAI_EHIP; the affected outputs are NaN) and clears the report. No
 * counterpart in the reference. */
int localai_hip_layer_error(void *workspace_dev, void *stream);

/* ---- decode-step attention mixers ---------------------------------------- */

/* Bytes of workspace localai_hip_attention_decode needs for any position
 * below max_seq (per-chunk partial results of the split-sequence decode); 0
 * for shapes without a kernel, -1 for invalid sizes. Calls on one workspace
 * must not overlap. */
int64_t localai_hip_attention_workspace_size(int64_t max_seq, int n_heads, int n_kv_heads, int head_dim);

/* Grouped-query attention of one decode token over one layer's KV cache,
 * the attention of engine/model.py:222-227 (`forward`) and, with gate_dev,
 * Qwen3.5's gated full attention (engine/qwen35.py:158-182):
 *   K[position], V[position] = k_new, v_new    (skipped when k_new_dev is NULL)
 *   out_h = softmax_s((q_h . K[s]) / sqrt(head_dim)) V[s],  s in [start, position]
 *   out_h *= 1 / (1 + exp(-clip(gate_h, -80, 80)))          (gate_dev not NULL)
 * Query head h reads kv head h / (n_heads / n_kv_heads) (np.repeat order,
 * engine/model.py:225); start = max(0, position + 1 - window) for window > 0,
 * else 0 (:223). Caches: fp32 [max_seq, n_kv_heads, head_dim]; q, gate and
 * out [n_heads, head_dim]; k_new, v_new [n_kv_heads, head_dim]; all 16-byte
 * aligned. head_dim 64, 128 or 256 with at most 16 / (head_dim / 64) query
 * heads per kv head; other shapes return LOCALAI_ETYPE. fp32 throughout:
 * within a few fp32 roundings of the reference's float32 einsum path. */
int localai_hip_attention_decode(const float *q_dev, const float *k_new_dev, const float *v_new_dev,
                                 float *k_cache_dev, float *v_cache_dev, int64_t position, int64_t max_seq,
                                 int n_heads, int n_kv_heads, int head_dim, int64_t window,
                                 const float *gate_dev, float *out_dev, void *workspace_dev,
                                 int64_t workspace_bytes, void *stream);

/* delta_net_step (engine/numba_kernels.py:11-45): one gated delta-rule step
 * of Qwen3.5's linear attention, per head h with S = state[h]
 * ([key_dim, value_dim] fp32, updated in place):
 *   S *= exp(decay[h]);  pred = S^T k[h];  delta = (v[h] - pred) * beta[h]
 *   S += k[h] delta^T;   core[h] = S^T q[h]
 * q, k [heads, key_dim]; v, core [heads, value_dim]; decay, beta [heads].
 * Every product and sum is rounded on its own in the reference loop's order,
 * so state and core equal the reference loop's bit for bit given the same
 * fp32 factor exp(decay). The kernel takes the correctly rounded exponential;
 * the reference's np.exp on float32 (engine/numba_kernels.py:25) can differ
 * from it in the last bit or two, and the results then differ at that level
 * (~1e-7 normwise). */
int localai_hip_delta_net_step(float *state_dev, const float *q_dev, const float *k_dev, const float *v_dev,
                               const float *decay_dev, const float *beta_dev, float *core_dev, int heads,
                               int key_dim, int value_dim, void *stream);

/* ---- ZAYA router (engine/zaya.py:274-307) -------------------------------- */

/* Everything of ZAYA's router after the first projection r0 = W_inp h
 * (engine/zaya.py:280-296), one workgroup: r = r0 + b_inp, then
 * r = r + prev * eda (skipped when prev and eda are NULL), state = r,
 * u = rmsnorm(r, eps) * norm_w, v1 = gelu(w_gate u + b_gate),
 * v2 = gelu(w_mlp2 v1 + b_mlp2), logits = w_mlp4 v2 + b_mlp4,
 * probs = softmax(logits), expert = argmax(probs + route_bias), the first
 * maximum. b_* are the projections' GGUF biases (NULL when absent,
 * engine/model.py:72-79). Matrices are fp32 device copies [rows, cols]
 * (w_gate [r1, r], w_mlp2 [r2, r1], w_mlp4 [routes, r2]); vectors up to
 * 4096, routes up to 512. GELU is exact (erf); the steps the reference
 * rounds in fp32 are separate fp32 operations. Outputs: state [r],
 * probs [routes], expert [1] (int32), and expert_w [1] = probs[expert] when
 * not NULL (the weight localai_hip_moe_experts1 takes), all device. */
int localai_hip_zaya_router(const float *r0_dev, const float *b_inp_dev, const float *prev_dev,
                            const float *eda_dev, const float *norm_w_dev, float eps, int64_t r,
                            const float *w_gate_dev, const float *b_gate_dev, int64_t r1,
                            const float *w_mlp2_dev, const float *b_mlp2_dev, int64_t r2,
                            const float *w_mlp4_dev, const float *b_mlp4_dev, int64_t routes,
                            const float *route_bias_dev, float *state_dev, float *probs_dev,
                            int32_t *expert_dev, float *expert_w_dev, void *stream);

/* gu_dev != NULL: y[i] = silu(gu[i]) * gu[n + i] (the expert SwiGLU on the
 * [gate; up] gate_up output, engine/zaya.py:304-305). gu_dev == NULL:
 * y[i] = x[i] * scale[0] with scale in device memory (the route probability,
 * :297-301 and :306). */
int localai_hip_zaya_scale(const float *gu_dev, const float *x_dev, int64_t n, const float *scale_dev,
                           float *y_dev, void *stream);

/* ---- MoE expert layer ---------------------------------------------------- */

/* Bytes of device workspace localai_hip_moe_forward needs for these sizes.
 * Calls that run at the same time need separate workspaces. */
int64_t localai_hip_moe_workspace_size(int64_t tokens, int64_t experts, int top_k,
                                       int64_t hidden, int64_t inter);

/* Where localai_hip_moe_forward leaves its routing tables in the workspace,
 * for inspection after the call: offs[0..11] = byte offsets of counts[E],
 * offsets[E + 1], active[E], n_active, perm[N], pos[N] (int32, N = tokens *
 * top_k; perm lists the assignments t * top_k + s in (expert, assignment)
 * order, pos is its inverse), then of the expert GEMM tile list tile_e,
 * tile_p0, tile_n (int32 [offs[10]] each) and n_tiles -- -1 below 32 tokens,
 * where the layer runs matvecs -- offs[10] = the tile list's capacity and
 * offs[11] = tokens per tile (0 below 32 tokens).
 * No counterpart in the reference (its tables live in Python lists). */
int localai_hip_moe_table_offsets(int64_t tokens, int64_t experts, int top_k, int64_t hidden,
                                  int64_t inter, int64_t *offs);

/* Top-k MoE FFN layer; composition of engine/zaya.py:274-307 (router, softmax,
 * expert selection with ties to the lower index, SiLU*up, weighted combine)
 * and engine/zaya.py:139-175 (expert = byte slice of a 3-D tensor):
 *   h_dev         [tokens, hidden] fp32
 *   router_w_dev  [experts, hidden] fp32;  router_b_dev [experts] fp32 or NULL
 *   gate_up       handle of [experts, 2*inter, hidden] (rows < inter = gate)
 *   down          handle of [experts, hidden, inter]
 *   out_dev       [tokens, hidden] fp32 = sum_s gate[t,s] * expert_s(h[t])
 *   topk_idx_dev  [tokens, top_k] int32, experts by (logit desc, index asc)
 *   topk_w_dev    [tokens, top_k] fp32, softmax over the selected logits
 * Router logits: exact fp64 products summed in a fixed order, rounded to fp32
 * once, so the selected experts are bit-reproducible. On return the workspace
 * begins with them: [tokens, experts] fp32, bias included.
 * Limits: experts <= 1024, 1 <= top_k <= min(16, experts), inter % 64 == 0;
 * h_dev and router_w_dev 16-byte aligned, workspace 256-byte aligned. */
int localai_hip_moe_forward(const float *h_dev, int64_t tokens, int64_t hidden,
                            const float *router_w_dev, const float *router_b_dev,
                            int64_t experts, int top_k, const localai_qmat *gate_up,
                            const localai_qmat *down, float *out_dev, int32_t *topk_idx_dev,
                            float *topk_w_dev, void *workspace_dev, int64_t workspace_bytes,
                            void *stream);

/* The expert part of the MoE layer for one token, with the chosen experts
 * already in device memory (written by a router kernel, so the host need not
 * read them): engine/zaya.py:297-306 for ZAYA's top-1 with its skip route.
 *   out_dev[hidden] = sum_s weight[s] * y_s, s < top_k (1 or 2), where
 *   y_s = h                                      if expert[s] == skip
 *       = down[e] (silu(gate) * up)(gate_up[e] h) otherwise (e = expert[s])
 * skip = -1 when every slot is an expert, else an index >= the expert count
 * (EARG for 0 <= skip < experts); an index in expert_dev outside
 * [0, experts) that is not skip makes that slot's rows of out NaN and is
 * reported by localai_hip_moe_error. One launch for gate_up and down
 * (plus a counter clear); the sum is the same whatever order the slots land.
 * Experts must be Q4_K, Q6_K or Q8_0 handles with the tile form (Q8_0:
 * hidden and inter multiples of 256), at most 32 blocks of 256 values a row
 * and inter % 64 == 0 (ETYPE otherwise: the caller then runs the matvec
 * path). Workspace: as
 * localai_hip_moe_workspace_size(1, experts, top_k, hidden, inter); h_dev
 * 16-byte and the workspace 256-byte aligned; out must not overlap h. */
int localai_hip_moe_experts1(const float *h_dev, int64_t hidden, const localai_qmat *gate_up,
                             const localai_qmat *down, int top_k, const int32_t *expert_dev,
                             const float *weight_dev, int32_t skip, float *out_dev, void *workspace_dev,
                             int64_t workspace_bytes, void *stream);

/* Bytes of the library's static device workspace (one per device, held
 * until the process ends) used by localai_hip_moe_forward_static. */
int64_t localai_hip_static_workspace_bytes(void);

/* localai_hip_moe_forward with the workspace taken from a static device array
 * inside the library (localai_hip_static_workspace_bytes() = 64 MiB per
 * device) instead of a caller buffer: it allocates nothing (no hipMalloc, no
 * hipFree), so callers that cannot allocate -- code under HIP graph capture,
 * serving loops that forbid allocation -- can run the MoE layer. Same
 * arguments, limits and results as localai_hip_moe_forward; sizes whose
 * workspace (localai_hip_moe_workspace_size) exceeds the static one are
 * LOCALAI_EARG; experts and sizes whose path would first build a handle's
 * row planes (below 32 tokens: Q8_0 rows of partial 256-value blocks, rows
 * over 64 blocks of 256; the ordinary entry builds them) are LOCALAI_ETYPE.
 * All calls on one device share its array: calls that overlap
 * in time on one device race, and the router logits the workspace holds
 * after a call are overwritten by the next. No counterpart in the reference. */
int localai_hip_moe_forward_static(const float *h_dev, int64_t tokens, int64_t hidden,
                                   const float *router_w_dev, const float *router_b_dev,
                                   int64_t experts, int top_k, const localai_qmat *gate_up,
                                   const localai_qmat *down, float *out_dev, int32_t *topk_idx_dev,
                                   float *topk_w_dev, void *stream);

/* Status of the last one-token fused expert launch that used this workspace
 * (localai_hip_moe_experts1, or localai_hip_moe_forward with one token and
 * top_k <= 2), which hands gate_up results to its down workgroups inside one
 * launch. Waits for `stream`, then reads the launch's error word: LOCALAI_EARG
 * if an expert index was outside [0, experts) and not the skip route,
 * LOCALAI_EHIP if a bounded wait ran out; either way the affected rows of out
 * are NaN. tokens / experts: as passed to that call. No counterpart in the
 * reference (its expert call raises synchronously, engine/native_quant.py:115-116). */
int localai_hip_moe_error(const void *workspace_dev, int64_t tokens, int64_t experts, void *stream);

/* Test control of the fused expert kernel's waits: at most spin_limit polls
 * per wait (<= 0: the default, seconds in all), and producers_count = 0 keeps
 * the gate_up workgroups from counting themselves done, so every wait runs
 * out and every workgroup still exits (the error path of
 * localai_hip_moe_error). Process-wide; (0, 1) restores the defaults. No
 * counterpart in the reference. */
int localai_hip_debug_fused_wait(int spin_limit, int producers_count);

/* ---- measurement -------------------------------------------------------- */

/* Read `bytes` (a multiple of 16) at src_dev once, as fast as the kernel can
 * stream them, and leave a fold of the data in out_dev[0] only in the
 * practically impossible case that it equals a fixed constant: the HBM read
 * floor the decode kernels are compared with (bench.py, hbm_read_floor). No
 * counterpart in the reference. */
int localai_hip_stream_read(const void *src_dev, int64_t bytes, uint32_t *out_dev, void *stream);

/* Run one expert GEMM of the MoE prefill path again (which = 0: gate_up with
 * SiLU*up, 1: down) on the routing tables and staged rows that the last
 * localai_hip_moe_forward over `tokens` tokens (>= 32, the expert GEMM path)
 * left in workspace_dev, with the same handles: that kernel timed alone.
 * Results land in the workspace only. No counterpart in the reference
 * (measurement: bench.py's qwen3_moe_prefill roofline). */
int localai_hip_moe_expert_gemm(const localai_qmat *gate_up, const localai_qmat *down, int64_t tokens,
                                int64_t experts, int top_k, void *workspace_dev, int64_t workspace_bytes, int which,
                                void *stream);

/* ---- host weight registration for the legacy exports -------------------- */

/* Declare [host, host+nbytes) immutable (e.g. a GGUF mmap). Legacy calls whose
 * `raw` lies inside a registered range reuse a cached device copy instead of
 * uploading the bytes on every call. */
int localai_hip_register_host(const void *host, size_t nbytes);
int localai_hip_unregister_host(const void *host);
/* Number of device copies the legacy exports hold for registered ranges
 * (diagnostics: a repeated call on a registered range adds none). No
 * reference counterpart. */
int64_t localai_hip_cache_entries(void);
/* Drop every cached device copy. */
int localai_hip_cache_clear(void);

/* ---- legacy exports: engine/native_quant.cpp:705-768 --------------------- */
/* out[rows] = W @ x.  engine/native_quant.cpp:705-738 */
void localai_q8_0_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, int threads);
void localai_q4_0_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, int threads);
void localai_q4k_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, int threads);
void localai_q5k_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, int threads);
void localai_q6k_matvec(const uint8_t *raw, const float *x, float *out, int rows, int cols, int threads);
/* out[rows, tokens] = W @ vectors^T (vectors [tokens, cols]).  engine/native_quant.cpp:744-768
 * Fewer than 32 tokens: the fp32 matvec; 32 tokens or more: the MFMA GEMM
 * (localai_hip_matmul: f16 operands, fp32 accumulation). */
void localai_q8_0_matmul(const uint8_t *raw, const float *vectors, float *out, int rows, int cols, int tokens, int threads);
void localai_q4_0_matmul(const uint8_t *raw, const float *vectors, float *out, int rows, int cols, int tokens, int threads);
void localai_q4k_matmul(const uint8_t *raw, const float *vectors, float *out, int rows, int cols, int tokens, int threads);
void localai_q5k_matmul(const uint8_t *raw, const float *vectors, float *out, int rows, int cols, int tokens, int threads);
void localai_q6k_matmul(const uint8_t *raw, const float *vectors, float *out, int rows, int cols, int tokens, int threads);

#ifdef __cplusplus
}
#endif
#endif /* LOCALAI_HIP_H */
