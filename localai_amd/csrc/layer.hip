// The matvec chain of one decode layer in one launch (engine/model.py:215-240,
// from the attention output of layer L to the attention inputs of layer L+1):
//
//   S1  o    = W_o att                                   (engine/model.py:229)
//   S2  x1   = pre + o;  u = norm(x1) * w_ffn            (:229-232, norm :82)
//       act  = silu(W_gate u) * (W_up u)                 (:232)
//   S3  d    = W_down act                                (:233)
//   S4  x2   = x1 + d;   v = norm(x2) * w_attn'          (:233, then :182 of L+1)
//       q, k, v' = W_q' v, W_k' v, W_v' v  (+ RoPE of q, k) (:183-185, :203-213)
//
// Each stage is a range of workgroups in one grid, in stage order: S1 tiles,
// S2 tiles, S3 tiles, S4 tiles. A workgroup of a later stage first requests
// its weights (they do not depend on the earlier stages) and only then waits
// until every workgroup of the previous stage has counted itself done, so
// the weight stream of the next stage runs while the previous stage's last
// workgroups finish: the chain streams its 139 MB (Llama-3-8B, Q4_K_M) as
// one launch instead of four launches, each with its ramp and tail.
// Workgroups start in id order, so every workgroup a wait depends on has
// started before the wait (the waits end).
//
// Per-tile arithmetic is the decode matvec of mfma_core.h (i8 MFMA, x as
// three int8 pieces, exact integer dot products, fp32 scales); the results
// equal localai_hip_matvec's for the same x. Data handed between stages
// (o, act, d) moves with device-coherent loads and stores (fused_sync.h).
//
// Workgroups (512 threads):
//   S1  one 16-row tile of W_o over the whole K (dim)
//   S2  gate tile i and up tile i (the SiLU*up epilogue needs both)
//   S3  one tile of W_down over one half of K (ffn); the two halves add onto
//       d, which the S1 workgroups cleared: two additions onto zero give the
//       same sum in either order
//   S4  one tile of W_q, W_k or W_v
// The sums of squares of the norms are fp64 in a fixed order, so every
// workgroup of a stage computes the same u bit for bit.
//
// Counters: a block of D1_WORDS words per stage (sharded completion counters,
// a done flag, an error word; fused_sync.h). The workgroup that completes S4
// returns every counter and flag to zero for the next launch (error words
// stay until localai_hip_layer_error reads them), so the workspace must be
// zero-filled once before its first launch.
#include <atomic>
#include <type_traits>

#include "fused_sync.h"
#include "internal.h"
#include "mfma_core.h"

// Phase marks of a workgroup (entry, weights requested, wait over, x ready,
// done); empty unless a profiling build defines it.
#ifndef LY_MARK
#define LY_MARK(phase)
#endif

namespace lq {

struct LyMat {
    const uint8_t *wt;   // tile form
    int type;            // LQ_Q4_K or LQ_Q6_K
    int rows;
};

struct LayerArgs {
    LyMat o, gate, up, down, q, k, v;
    int dim, ffn;            // hidden size (cols of o / gate / up / q / k / v), intermediate size
    int nbd, nbf, half;      // super-blocks per row of dim / ffn; super-blocks in the first half of ffn
    const float *pre, *att, *w_ffn, *w_attn;
    float eps;
    const float *rope_cos, *rope_sin;   // [rope_half] or null
    int head_dim, rope_half;
    float *x_out, *q_out, *k_out, *v_out;
    float *o_buf, *act_buf, *d_buf;
    uint32_t *sync;          // 4 stage blocks of D1_WORDS
    int n1, n2, n3, n4;      // workgroups per stage
    int tq, tk;              // tiles of W_q and W_k (S4 layout: q, k, v)
    int spin, count;
};

constexpr int LY_THREADS = 512;

// device-coherent 16-byte load (two 8-byte relaxed device-scope loads)
__device__ __forceinline__ float4 ly_get4(const float *p) {
    const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
    const uint64_t lo = d1_get(q), hi = d1_get(q + 1);
    return make_float4(__builtin_bit_cast(float, (uint32_t)lo), __builtin_bit_cast(float, (uint32_t)(lo >> 32)),
                       __builtin_bit_cast(float, (uint32_t)hi), __builtin_bit_cast(float, (uint32_t)(hi >> 32)));
}

// Whole workgroup: wait for stage block `blk` to be done. One thread polls
// (at once, then about every 500 cycles, at most `spin` polls).
__device__ __forceinline__ bool ly_wait(uint32_t *blk, int *flag, int spin) {
    if (threadIdx.x == 0) {
        int ok = 0;
        for (int n = 0; n < spin; ++n) {
            if (d1_get(blk + D1_DONE) != 0u) {
                ok = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
        if (!ok) d1_error(blk, D1_ERR_WAIT);
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

// x1 = pre + o (and + d when WITH_D), u = x1 * (1 / sqrt(mean(x1^2) + eps)) * w
// into xs (LDS, dim floats); o and d are read device-coherent. Returns after a
// barrier. The sum of squares is fp64: per thread in index order, then the
// 64 lanes in a fixed tree, then the waves in order.
template <bool WITH_D>
__device__ __forceinline__ void ly_norm_input(const LayerArgs &a, const float *w, float *xs, double *red,
                                              float *x_keep) {
    const int tid = threadIdx.x, n4 = a.dim >> 2;
    double ss = 0.0;
    for (int c = tid; c < n4; c += LY_THREADS) {
        const float4 p = reinterpret_cast<const float4 *>(a.pre)[c];
        const float4 o = ly_get4(a.o_buf + 4 * c);
        float4 x = make_float4(__fadd_rn(p.x, o.x), __fadd_rn(p.y, o.y), __fadd_rn(p.z, o.z), __fadd_rn(p.w, o.w));
        if (WITH_D) {
            const float4 d = ly_get4(a.d_buf + 4 * c);
            x = make_float4(__fadd_rn(x.x, d.x), __fadd_rn(x.y, d.y), __fadd_rn(x.z, d.z), __fadd_rn(x.w, d.w));
        }
        reinterpret_cast<float4 *>(xs)[c] = x;
        if (x_keep) reinterpret_cast<float4 *>(x_keep)[c] = x;
        ss += (double)x.x * x.x;
        ss += (double)x.y * x.y;
        ss += (double)x.z * x.z;
        ss += (double)x.w * x.w;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < LY_THREADS / 64; ++i) tot += red[i];
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)(tot / (double)a.dim), a.eps)));
    for (int c = tid; c < a.dim; c += LY_THREADS) xs[c] = __fmul_rn(__fmul_rn(xs[c], inv), w[c]);
    __syncthreads();
}

// x values of the wave's super-blocks from an fp32 vector in LDS
template <int SPW>
__device__ __forceinline__ void ly_x_from_lds(float4 (&xv)[SPW], const float *xs, int nb, int sb0, int lane) {
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;
        xv[k] = reinterpret_cast<const float4 *>(xs)[64 * sb + lane];
    }
}

template <int TYPE, int SPW, int RT>
__device__ __forceinline__ void ly_load(MtW<TYPE> (&w)[RT][SPW], const uint8_t *const (&tile)[RT], int nb) {
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
#pragma unroll
    for (int t = 0; t < RT; ++t) mt_load_tile<TYPE, SPW>(w[t], tile[t], nb, sb0, nsb, lane);
}

// The dot products of the RT tiles in w with x (xv) over nb super-blocks;
// fin (LDS) holds row n of tile t at 16 t + n after the call.
template <int TYPE, int SPW, int RT>
__device__ __forceinline__ void ly_dot(const MtW<TYPE> (&w)[RT][SPW], const float4 (&xv)[1][SPW], int nb,
                                       uint8_t *smem, float *&fin) {
    const int nsb = mt_nsb(nb, wave_id() * SPW, SPW);
    mt_pass<TYPE, SPW, RT, 1>(w, xv, nsb, smem, fin);
}

// Workgroup r of stage S1..S3 counts itself done (unless the test control
// says not to); S4's last workgroup resets every counter block. The host
// also clears the blocks before each launch (ly_clear_kernel), so a count
// that arrives after that reset (a wait that ran out) is not carried into
// the next launch; the error words then report the last launch.
__device__ __forceinline__ void ly_done(const LayerArgs &a, int stage, int r, int n, int *flag) {
    d1_drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = (a.count || stage == 3) && d1_count(a.sync + stage * D1_WORDS, r, n);
        *flag = last && stage == 3;
    }
    __syncthreads();
    // the words a launch changes: D1_NCNT counters, the full counter and
    // the done flag of each stage block
    const int i = threadIdx.x;
    if (*flag && i < 4 * (D1_NCNT + 2)) {
        const int s = i / (D1_NCNT + 2), c = i % (D1_NCNT + 2);
        const int word = c < D1_NCNT ? c * D1_LINE : c == D1_NCNT ? D1_FULL : D1_DONE;
        d1_put(a.sync + s * D1_WORDS + word, 0u);
    }
}

// ---------------------------------------------------------------- stages

template <int SPWD>
__device__ __forceinline__ void ly_stage_o(const LayerArgs &a, int j, uint8_t *smem, int *flag) {
    LY_MARK(0);
    const int lane = lane_id(), sb0 = wave_id() * SPWD;
    float4 xv[1][SPWD];
    mt_load_x<SPWD>(xv[0], a.att, a.nbd, sb0, lane);
    const uint8_t *tile[1] = {a.o.wt + (int64_t)j * a.nbd * mt_block_bytes(a.o.type)};
    float *fin;
    if (a.o.type == LQ_Q6_K) {
        MtW<LQ_Q6_K> w[1][SPWD];
        ly_load<LQ_Q6_K, SPWD, 1>(w, tile, a.nbd);
        ly_dot<LQ_Q6_K, SPWD, 1>(w, xv, a.nbd, smem, fin);
    } else {
        MtW<LQ_Q4_K> w[1][SPWD];
        ly_load<LQ_Q4_K, SPWD, 1>(w, tile, a.nbd);
        ly_dot<LQ_Q4_K, SPWD, 1>(w, xv, a.nbd, smem, fin);
    }
    const int i = threadIdx.x, row = j * MT_ROWS + i;
    if (i < MT_ROWS && row < a.o.rows) d1_put(a.o_buf + row, fin[i]);
    // clear this workgroup's share of d (S3 adds onto it)
    LY_MARK(3);
    const int per = (a.dim + a.n1 - 1) / a.n1;
    for (int c = j * per + i; c < (j + 1) * per && c < a.dim; c += LY_THREADS) d1_put(a.d_buf + c, 0.0f);
    ly_done(a, 0, j, a.n1, flag);
    LY_MARK(4);
}

template <int SPWD>
__device__ __forceinline__ void ly_stage_gu(const LayerArgs &a, int j, uint8_t *smem, int *flag, double *red) {
    const int lane = lane_id(), sb0 = wave_id() * SPWD;
    const int64_t toff = (int64_t)j * a.nbd * mt_block_bytes(a.gate.type);
    const uint8_t *tile[2] = {a.gate.wt + toff, a.up.wt + toff};
    float *xs = reinterpret_cast<float *>(smem);
    uint8_t *pass = smem + (size_t)a.dim * 4;
    float *fin;
    auto body = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        MtW<T> w[2][SPWD];
        LY_MARK(0);
        ly_load<T, SPWD, 2>(w, tile, a.nbd);
        LY_MARK(1);
        const bool ok = ly_wait(a.sync + 0 * D1_WORDS, flag, a.spin);
        LY_MARK(2);
        ly_norm_input<false>(a, a.w_ffn, xs, red, nullptr);
        LY_MARK(3);
        float4 xv[1][SPWD];
        ly_x_from_lds<SPWD>(xv[0], xs, a.nbd, sb0, lane);
        ly_dot<T, SPWD, 2>(w, xv, a.nbd, pass, fin);
        const int i = threadIdx.x, row = j * MT_ROWS + i;
        if (i < MT_ROWS && row < a.gate.rows)
            d1_put(a.act_buf + row, ok ? __fmul_rn(silu(fin[i]), fin[MT_ROWS + i]) : __builtin_nanf(""));
    };
    if (a.gate.type == LQ_Q6_K) body(std::integral_constant<int, LQ_Q6_K>{});
    else body(std::integral_constant<int, LQ_Q4_K>{});
    ly_done(a, 1, j, a.n2, flag);
    LY_MARK(4);
}

template <int SPWF>
__device__ __forceinline__ void ly_stage_down(const LayerArgs &a, int j, uint8_t *smem, int *flag) {
    const int lane = lane_id(), sb0 = wave_id() * SPWF;
    const int t = j >> 1, h = j & 1;
    const int k0 = h * a.half, nbl = h ? a.nbf - a.half : a.half;
    const int bb = mt_block_bytes(a.down.type);
    const uint8_t *tile[1] = {a.down.wt + ((int64_t)t * a.nbf + k0) * bb};
    float *fin;
    auto body = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        MtW<T> w[1][SPWF];
        LY_MARK(0);
        ly_load<T, SPWF, 1>(w, tile, nbl);
        LY_MARK(1);
        const bool ok = ly_wait(a.sync + 1 * D1_WORDS, flag, a.spin);
        LY_MARK(2);
        float4 xv[1][SPWF];
        d1_load_x<SPWF>(xv[0], a.act_buf + (int64_t)k0 * 256, nbl, sb0, lane);
        LY_MARK(3);
        ly_dot<T, SPWF, 1>(w, xv, nbl, smem, fin);
        const int i = threadIdx.x, row = t * MT_ROWS + i;
        if (i < MT_ROWS && row < a.down.rows)
            __hip_atomic_fetch_add(a.d_buf + row, ok ? fin[i] : __builtin_nanf(""), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    };
    if (a.down.type == LQ_Q6_K) body(std::integral_constant<int, LQ_Q6_K>{});
    else body(std::integral_constant<int, LQ_Q4_K>{});
    ly_done(a, 2, j, a.n3, flag);
    LY_MARK(4);
}

template <int SPWD>
__device__ __forceinline__ void ly_stage_qkv(const LayerArgs &a, int j, uint8_t *smem, int *flag, double *red) {
    const int lane = lane_id(), sb0 = wave_id() * SPWD;
    const int m = j < a.tq ? 0 : j < a.tq + a.tk ? 1 : 2;
    const int t = m == 0 ? j : m == 1 ? j - a.tq : j - a.tq - a.tk;
    const LyMat &M = m == 0 ? a.q : m == 1 ? a.k : a.v;
    float *out = m == 0 ? a.q_out : m == 1 ? a.k_out : a.v_out;
    const uint8_t *tile[1] = {M.wt + (int64_t)t * a.nbd * mt_block_bytes(M.type)};
    float *xs = reinterpret_cast<float *>(smem);
    uint8_t *pass = smem + (size_t)a.dim * 4;
    float *fin;
    bool ok = true;
    auto body = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        MtW<T> w[1][SPWD];
        LY_MARK(0);
        ly_load<T, SPWD, 1>(w, tile, a.nbd);
        LY_MARK(1);
        ok = ly_wait(a.sync + 2 * D1_WORDS, flag, a.spin);
        LY_MARK(2);
        ly_norm_input<true>(a, a.w_attn, xs, red, j == 0 ? a.x_out : nullptr);
        LY_MARK(3);
        float4 xv[1][SPWD];
        ly_x_from_lds<SPWD>(xv[0], xs, a.nbd, sb0, lane);
        ly_dot<T, SPWD, 1>(w, xv, a.nbd, pass, fin);
    };
    if (M.type == LQ_Q6_K) body(std::integral_constant<int, LQ_Q6_K>{});
    else body(std::integral_constant<int, LQ_Q4_K>{});
    const int i = threadIdx.x, row = t * MT_ROWS + i;
    if (i < MT_ROWS && row < M.rows) {
        float y = fin[i];
        if (m < 2 && a.rope_cos) {   // adjacent-pair RoPE (engine/model.py:205-210)
            const int dd = row % a.head_dim, pj = dd >> 1;
            if (pj < a.rope_half) {
                const float other = fin[i ^ 1], c = a.rope_cos[pj], s = a.rope_sin[pj];
                y = (dd & 1) ? __fadd_rn(__fmul_rn(other, s), __fmul_rn(y, c))
                             : __fsub_rn(__fmul_rn(y, c), __fmul_rn(other, s));
            }
        }
        out[row] = ok ? y : __builtin_nanf("");
    }
    ly_done(a, 3, j, a.n4, flag);
    LY_MARK(4);
}

template <int SPWD, int SPWF>
__global__ __launch_bounds__(LY_THREADS) void layer_chain_kernel(LayerArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int flag;
    __shared__ double red[LY_THREADS / 64];
    int b = blockIdx.x;
    if (b < a.n1) {
        ly_stage_o<SPWD>(a, b, smem, &flag);
        return;
    }
    b -= a.n1;
    if (b < a.n2) {
        ly_stage_gu<SPWD>(a, b, smem, &flag, red);
        return;
    }
    b -= a.n2;
    if (b < a.n3) {
        ly_stage_down<SPWF>(a, b, smem, &flag);
        return;
    }
    ly_stage_qkv<SPWD>(a, b - a.n3, smem, &flag, red);
}

// ---------------------------------------------------------------- host side

static size_t ly_align(size_t x) { return (x + 255) & ~(size_t)255; }

// sync blocks | o [dim] | d [dim] | act [ffn] | per-tile sums of squares
// [MT_SSQ] (dim / 16 of them written, the rest stays zero). The four-launch
// form keeps x1 in o and x * w in d.
size_t layer_workspace_bytes(int64_t dim, int64_t ffn) {
    return ly_align(4 * D1_WORDS * 4) + ly_align(dim * 4) * 2 + ly_align(ffn * 4) + ly_align(MT_SSQ * 4);
}

static std::atomic<int> g_ly_spin{D1_SPIN_LIMIT}, g_ly_count{1}, g_ly_mode{0};

int set_layer_mode(int one_launch) {
    g_ly_mode.store(one_launch ? 1 : 0);
    return LOCALAI_OK;
}

// The chain as four launches, the glue fused into the matvec kernels
// (gemv_mfma.hip), each launch waiting for the one before it on the stream
// (nothing waits on the device):
//   o       x1 = pre + W_o att; also xs = x1 * w_ffn and x1's per-tile sums
//           of squares
//   gate/up act = silu(inv W_gate xs) * (inv W_up xs), inv = the norm factor
//           of x1 from its sums of squares; a workgroup holds gate tile i and
//           up tile i
//   down    x_out = x1 + W_down act; also xs = x_out * w_attn and x_out's sums
//           of squares
//   q/k/v   inv' (W_q xs), inv' (W_k xs), inv' (W_v xs), RoPE of q and k
static int ly_launch_glue(const localai_qmat *const *m, const float *pre, const float *att, const float *w_ffn,
                          const float *w_attn, float eps, const float *rope_cos, const float *rope_sin,
                          int head_dim, int rope_half, float *x_out, float *q_out, float *k_out, float *v_out,
                          float *x1, float *xs, float *act, float *ssq, hipStream_t s) {
    const int64_t dim = m[0]->g.rows;
    MtGlue gl{};
    gl.res = pre;
    gl.ssq_out = ssq;
    gl.w_next = w_ffn;
    gl.y_next = xs;
    if (int st = launch_matvec_mfma_glue(m[0]->g, m[0]->tiles, att, x1, MT_PRO_X, MT_EPI_RES, gl, s)) return st;
    gl = MtGlue{};
    gl.ssq_in = ssq;
    gl.n = (int)dim;
    gl.eps = eps;
    gl.Wt2 = m[2]->tiles;
    if (int st = launch_matvec_mfma_glue(m[1]->g, m[1]->tiles, xs, act, MT_PRO_NORM, MT_EPI_SILU, gl, s)) return st;
    gl = MtGlue{};
    gl.res = x1;
    gl.ssq_out = ssq;   // the norm before it has read ssq and xs (stream order)
    gl.w_next = w_attn;
    gl.y_next = xs;
    if (int st = launch_matvec_mfma_glue(m[3]->g, m[3]->tiles, act, x_out, MT_PRO_X, MT_EPI_RES, gl, s)) return st;
    gl = MtGlue{};
    gl.ssq_in = ssq;
    gl.n = (int)dim;
    gl.eps = eps;
    gl.cos = rope_cos;
    gl.sin = rope_sin;
    gl.head_dim = rope_cos ? head_dim : 2;
    gl.rope_half = rope_cos ? rope_half : 0;
    gl.rope_jobs = rope_cos ? 2 : 0;
    const lq_geom *g[3] = {&m[4]->g, &m[5]->g, &m[6]->g};
    const uint8_t *w[3] = {m[4]->tiles, m[5]->tiles, m[6]->tiles};
    float *y[3] = {q_out, k_out, v_out};
    return launch_matvec_mfma_many_glue(3, g, w, xs, y, MT_PRO_NORM, rope_cos ? MT_EPI_ROPE : MT_EPI_Y, gl, s);
}

int set_layer_wait(int spin, int count) {
    g_ly_spin.store(spin > 0 ? spin : D1_SPIN_LIMIT);
    g_ly_count.store(count ? 1 : 0);
    return LOCALAI_OK;
}

// error bits of the four stage blocks (after the stream has finished); clears them
int layer_error_word(void *ws, hipStream_t s, uint32_t *word) {
    uint32_t *sync = (uint32_t *)ws;
    LQ_HIP(hipStreamSynchronize(s));
    uint32_t w = 0, e[4];
    for (int i = 0; i < 4; ++i) {
        LQ_HIP(hipMemcpy(&e[i], sync + i * D1_WORDS + D1_ERROR, 4, hipMemcpyDeviceToHost));
        w |= e[i];
    }
    if (w) {
        // a failed launch may also have left counters behind: clear the blocks
        LQ_HIP(hipMemset(sync, 0, 4 * D1_WORDS * 4));
    }
    *word = w;
    return LOCALAI_OK;
}

static int ly_spw(int nb) { return (nb + 7) / 8; }

// Zeroes the four stage blocks ahead of a one-launch chain (a kernel, not a
// memset, so the call can be captured in a graph): a launch whose wait ran
// out may have left a late count behind after S4's reset, and the next
// launch must not start from it.
__global__ void ly_clear_kernel(uint32_t *__restrict__ sync, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) sync[i] = 0u;
}

int launch_layer_chain(const localai_qmat *const *m, const float *pre, const float *att, const float *w_ffn,
                       const float *w_attn, float eps, const float *rope_cos, const float *rope_sin, int head_dim,
                       int rope_half, float *x_out, float *q_out, float *k_out, float *v_out, void *ws,
                       hipStream_t s) {
    // m: o, gate, up, down, q, k, v
    const int64_t dim = m[0]->g.rows, ffn = m[1]->g.rows;
    LayerArgs a{};
    LyMat *dst[7] = {&a.o, &a.gate, &a.up, &a.down, &a.q, &a.k, &a.v};
    for (int i = 0; i < 7; ++i) {
        dst[i]->wt = m[i]->tiles;
        dst[i]->type = m[i]->g.type;
        dst[i]->rows = (int)m[i]->g.rows;
    }
    a.dim = (int)dim;
    a.ffn = (int)ffn;
    a.nbd = (int)(dim / 256);
    a.nbf = (int)(ffn / 256);
    a.half = (a.nbf + 1) / 2;
    a.pre = pre;
    a.att = att;
    a.w_ffn = w_ffn;
    a.w_attn = w_attn;
    a.eps = eps;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.head_dim = head_dim;
    a.rope_half = rope_half;
    a.x_out = x_out;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    uint8_t *p = (uint8_t *)ws;
    a.sync = (uint32_t *)p;
    p += ly_align(4 * D1_WORDS * 4);
    a.o_buf = (float *)p;
    p += ly_align(dim * 4);
    a.d_buf = (float *)p;
    p += ly_align(dim * 4);
    a.act_buf = (float *)p;
    p += ly_align(ffn * 4);
    // the glued matvecs take rows of at most 8192 (norm prologue) and 18432
    // (down) values; larger layers run as one launch
    if (g_ly_mode.load() == 0 && dim <= 8192 && ffn <= 18432)
        return ly_launch_glue(m, pre, att, w_ffn, w_attn, eps, rope_cos, rope_sin, head_dim, rope_half, x_out, q_out,
                              k_out, v_out, a.o_buf, a.d_buf, a.act_buf, (float *)p, s);
    a.n1 = (int)(dim / MT_ROWS);
    a.n2 = (int)(ffn / MT_ROWS);
    a.n3 = 2 * (int)(dim / MT_ROWS);
    a.tq = (int)((m[4]->g.rows + MT_ROWS - 1) / MT_ROWS);
    a.tk = (int)((m[5]->g.rows + MT_ROWS - 1) / MT_ROWS);
    a.n4 = a.tq + a.tk + (int)((m[6]->g.rows + MT_ROWS - 1) / MT_ROWS);
    a.spin = g_ly_spin.load();
    a.count = g_ly_count.load();
    const int spwd = ly_spw(a.nbd), spwf = ly_spw(a.half);
    const size_t lds_d6 = (size_t)dim * 4 + mt_lds_bytes(LQ_Q6_K, 8, spwd, 1, 2);
    const size_t lds_f6 = mt_lds_bytes(LQ_Q6_K, 8, spwf, 1, 1);
    const size_t lds = lds_d6 > lds_f6 ? lds_d6 : lds_f6;
    if (lds > max_lds_per_block()) return fail(LOCALAI_ETYPE, "layer chain: dim too large for the LDS");
    const dim3 grid((unsigned)(a.n1 + a.n2 + a.n3 + a.n4)), block(LY_THREADS);
    hipLaunchKernelGGL(ly_clear_kernel, dim3(1), dim3(256), 0, s, a.sync, 4 * D1_WORDS);
    LQ_HIP(hipGetLastError());
#define LY_L(D, F)                                                                                  \
    if (spwd == D && spwf == F) {                                                                   \
        hipLaunchKernelGGL((layer_chain_kernel<D, F>), grid, block, lds, s, a);                     \
        LQ_HIP(hipGetLastError());                                                                  \
        return LOCALAI_OK;                                                                          \
    }
    LY_L(2, 4) LY_L(2, 3) LY_L(2, 2) LY_L(1, 1) LY_L(1, 2) LY_L(1, 3) LY_L(3, 4) LY_L(3, 3)
#undef LY_L
    return fail(LOCALAI_ETYPE, "layer chain: no kernel for this dim / ffn (super-blocks per wave)");
}

}  // namespace lq
