// Top-k mixture-of-experts FFN layer on quantized expert tensors.
//
// Semantics (generalising engine/zaya.py:274-307 from top-1 to top-k):
//   logits[t, e] = canonical fp32 router logit (+ bias[e])
//   idx[t, :]    = k largest logits, ties to the lower expert index
//                  (np.argmax rule, engine/zaya.py:296)
//   gate[t, :]   = softmax over the k selected logits (renormalised top-k)
//   out[t]       = sum_s gate[t, s] * W_down[e_s] @ (silu(g) * u),
//                  [g; u] = W_gate_up[e_s] @ h[t]   (first half gate, engine/zaya.py:303-306)
//   silu(g)      = g / (1 + exp(-clip(g, -80, 80)))  (engine/zaya.py:305)
//
// Kernels (one stream, in order):
//   route     one workgroup per token: router logits, top-k, gates
//   permute   one workgroup: expert histogram, exclusive scan, stable
//             expert-major permutation of the T*k assignments (LDS)
//   gate_up   grouped matvec over the active experts, one workgroup per
//             (64-row gate tile + matching up tile, expert); SiLU*up fused
//   down      grouped matvec over the active experts
//   combine   gate-weighted sum of each token's k expert outputs (fixed order)
//
// Router logits are bit-reproducible: each is a sum of exact fp64 products
// h*w in a fixed order (lane l sums elements l, l+64, ...; then a pairwise
// tree over the 64 lanes), rounded to fp32 once.
#include <math.h>

#include "gemv_core.h"
#include "internal.h"

namespace lq {

struct MoeTables {
    float *logits;      // [T, E]
    int32_t *counts;    // [E]
    int32_t *offsets;   // [E + 1]
    int32_t *active;    // [E] active experts, ascending
    int32_t *n_active;  // [1]
    int32_t *perm;      // [N] assignment ids (t*k + s) in expert-major order
    int32_t *pos;       // [N] position of assignment a in perm
    float *act;         // [N, I] silu(gate)*up per assignment, perm order
    float *ysl;         // [N, H] expert outputs per assignment, perm order
};

// ------------------------------------------------------------------ route

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ h, int H,
                                                        const float *__restrict__ rw,
                                                        const float *__restrict__ rb, int E, int k,
                                                        float *__restrict__ logits,
                                                        int32_t *__restrict__ topk_idx,
                                                        float *__restrict__ topk_w) {
    extern __shared__ float lg[];          // E logits of this token
    const int t = blockIdx.x;
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    const float *ht = h + (int64_t)t * H;
    for (int e = w; e < E; e += nw) {
        const float *we = rw + (int64_t)e * H;
        double s = 0.0;
        for (int i = lane; i < H; i += 64) s = __builtin_fma((double)ht[i], (double)we[i], s);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) {
            float v = (float)s;
            if (rb) v = v + rb[e];
            lg[e] = v;
            logits[(int64_t)t * E + e] = v;
        }
    }
    __syncthreads();
    if (w != 0) return;
    // lane l owns experts l, l+64, ...; bit j of `taken` marks expert l+64j as selected
    uint32_t taken = 0;
    float myv = -INFINITY;
    int myi = 0;
    for (int r = 0; r < k; ++r) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int e = lane, j = 0; e < E; e += 64, ++j)
            if (!((taken >> j) & 1u) && better(lg[e], e, bv, bi)) { bv = lg[e]; bi = e; }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == r) { myv = bv; myi = bi; }
    }
    const float vmax = __shfl(myv, 0, 64);
    const float ex = lane < k ? expf(myv - vmax) : 0.0f;
    float z = ex;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);
    if (lane < k) {
        topk_idx[(int64_t)t * k + lane] = myi;
        topk_w[(int64_t)t * k + lane] = ex / z;
    }
}

// ---------------------------------------------------------------- permute

// Stable counting sort of N assignments by expert in one workgroup of 1024
// threads: per-wave histograms, exclusive offsets in (expert, wave) order,
// then each wave places its contiguous range in order.
__global__ __launch_bounds__(1024) void moe_permute_kernel(const int32_t *__restrict__ idx, int N, int E,
                                                           MoeTables tb) {
    extern __shared__ int ws[];            // cnt[16][E], run[16][E], total[E], off[E+1]
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    int *cnt = ws;
    int *run = ws + 16 * E;
    int *total = ws + 32 * E;
    int *off = ws + 33 * E;
    for (int i = threadIdx.x; i < 33 * E + E + 1; i += blockDim.x) ws[i] = 0;
    __syncthreads();
    const int per = (N + nw - 1) / nw;
    const int a0 = w * per, a1 = min(N, a0 + per);
    for (int a = a0 + lane; a < a1; a += 64) atomicAdd(&cnt[w * E + idx[a]], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int r = 0;
        for (int ww = 0; ww < nw; ++ww) {
            int c = cnt[ww * E + e];
            cnt[ww * E + e] = r;           // exclusive within the expert
            r += c;
        }
        total[e] = r;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int o = 0, na = 0;
        for (int e = 0; e < E; ++e) {
            off[e] = o;
            tb.offsets[e] = o;
            tb.counts[e] = total[e];
            if (total[e] > 0) tb.active[na++] = e;
            o += total[e];
        }
        off[E] = o;
        tb.offsets[E] = o;
        tb.n_active[0] = na;
    }
    __syncthreads();
    for (int base = a0; base < a1; base += 64) {
        const int a = base + lane;
        const bool live = a < a1;
        const int e = live ? idx[a] : -1;
        int rank = 0;
        bool last_of_e = true;
        for (int j = 0; j < 64; ++j) {
            int ej = __shfl(e, j, 64);
            if (ej == e && j < lane) ++rank;
            if (ej == e && j > lane) last_of_e = false;
        }
        if (live) {
            const int p = off[e] + cnt[w * E + e] + run[w * E + e] + rank;
            tb.perm[p] = a;
            tb.pos[a] = p;
        }
        __builtin_amdgcn_wave_barrier();
        if (live && last_of_e) run[w * E + e] += rank + 1;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        __builtin_amdgcn_wave_barrier();
    }
}

// --------------------------------------------------------- grouped matvec

__device__ __forceinline__ float silu(float g) {
    const float c = fminf(fmaxf(g, -80.0f), 80.0f);
    return g / (1.0f + expf(-c));
}

constexpr int MOE_R = 4;   // rows per lane group per matrix half

// One workgroup: a tile of MOE_R * G rows (G = 64 / LPR lane groups) of one
// expert for NT of its tokens. gate_up: rows r of the gate half and
// r + inter of the up half (one x staging, one reduction), written as
// silu(g) * u; down: rows r of the down matrix. With LPR = 64 the waves
// split the K units. Not inlined: the NT = 1 and NT = 2 bodies would
// otherwise share one register budget.
template <int T, int NT, bool GATE_UP, int LPR>
__device__ __noinline__ void expert_chunk(const uint8_t *__restrict__ Wexp, const lq_geom &g, int64_t row0,
                                          const float *const *xrow, float *red, float4 *xlds,
                                          float *__restrict__ outp, int64_t out_stride) {
    const int w = wave_id(), nw = blockDim.x >> 6;
    const int64_t half = GATE_UP ? g.rows / 2 : g.rows;
    constexpr int SETS = GATE_UP ? 2 : 1;
    constexpr int RT = MOE_R * SETS;     // register rows per lane
    constexpr int G = 64 / LPR;
    int vi;
    bool writer;
    const float v = wave_rows<T, NT, 1, RT, LPR, SETS>(Wexp, g, row0, half + row0, GATE_UP ? g.rows : half, w,
                                                       xrow, xlds + w * NT * 16 * LPR, vi, writer);
    // red[(w * G + group) * RT * NT + value]; value r * NT + t, set-1 rows
    // (up half) after the MOE_R * NT set-0 values
    if (writer) red[(w * G + lane_id() / LPR) * RT * NT + vi] = v;
    __syncthreads();
    const int i = threadIdx.x;
    if (i < G * MOE_R * NT) {
        const int gi = i / (MOE_R * NT), j = i % (MOE_R * NT);
        float sa = 0.0f, sb = 0.0f;
        for (int k = 0; k < nw; ++k) {
            sa += red[(k * G + gi) * RT * NT + j];
            if (GATE_UP) sb += red[(k * G + gi) * RT * NT + MOE_R * NT + j];
        }
        const int r = j / NT, t = j % NT;
        const int64_t row = row0 + gi * MOE_R + r;
        if (row < half) outp[t * out_stride + row] = GATE_UP ? silu(sa) * sb : sa;
    }
    __syncthreads();
}

template <int T, bool GATE_UP, int LPR>
__global__ __launch_bounds__(256) void moe_grouped_kernel(const uint8_t *__restrict__ Wall, lq_geom g,
                                                          MoeTables tb, const float *__restrict__ xsrc,
                                                          int64_t x_stride, int k) {
    extern __shared__ float4 xlds[];            // 2 * 16 * LPR float4 per wave (NT <= 2)
    __shared__ float red[4 * 2 * MOE_R * 2];    // [waves x groups][rows of both sets][NT <= 2]
    const int slot = blockIdx.y;
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int n = tb.counts[e], base = tb.offsets[e];
    const uint8_t *Wexp = Wall + (int64_t)e * g.matrix_bytes;
    const int64_t row0 = (int64_t)blockIdx.x * MOE_R * (64 / LPR);
    // gate_up: x = token rows of h, out = act rows [p, inter]; down: x = act rows, out = ysl rows [p, H]
    const int64_t out_stride = GATE_UP ? g.rows / 2 : g.rows;
    float *outbase = GATE_UP ? tb.act : tb.ysl;
    for (int t0 = 0; t0 < n;) {
        const int nt = n - t0 >= 2 ? 2 : 1;
        const float *xrow[2];
        for (int t = 0; t < 2; ++t) {
            const int p = base + t0 + (t < nt ? t : 0);
            const int64_t src = GATE_UP ? (int64_t)(tb.perm[p] / k) : (int64_t)p;
            xrow[t] = xsrc + src * x_stride;
        }
        float *outp = outbase + (int64_t)(base + t0) * out_stride;
        if (nt == 2) expert_chunk<T, 2, GATE_UP, LPR>(Wexp, g, row0, xrow, red, xlds, outp, out_stride);
        else expert_chunk<T, 1, GATE_UP, LPR>(Wexp, g, row0, xrow, red, xlds, outp, out_stride);
        t0 += nt;
    }
}

// ---------------------------------------------------------------- combine

// out[t, :] = sum_j topk_w[t, j] * ysl[pos[t*k + j], :], slots in top-k order
__global__ void moe_combine_kernel(const float *__restrict__ ysl, const int32_t *__restrict__ pos,
                                   const float *__restrict__ topk_w, int k, int H, float *__restrict__ out) {
    const int t = blockIdx.y;
    const int hcol = blockIdx.x * blockDim.x + threadIdx.x;
    if (hcol >= H) return;
    float s = 0.0f;
    for (int j = 0; j < k; ++j) {
        const int p = pos[t * k + j];
        s = __builtin_fmaf(topk_w[t * k + j], ysl[(int64_t)p * H + hcol], s);
    }
    out[(int64_t)t * H + hcol] = s;
}

// ---------------------------------------------------------------- host side

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t moe_workspace_bytes(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const int64_t N = T * k;
    size_t s = 0;
    s += align256(T * E * 4);                                        // logits
    s += align256(E * 4) * 2 + align256((E + 1) * 4) + align256(4);  // counts, offsets, active, n_active
    s += align256(N * 4) * 2;                                        // perm, pos
    s += align256(N * I * 4);                                        // act
    s += align256(N * H * 4);                                        // ysl
    return s;
}

static MoeTables carve(void *ws, int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const int64_t N = T * k;
    uint8_t *p = (uint8_t *)ws;
    MoeTables tb;
    auto take = [&](size_t n) { uint8_t *q = p; p += align256(n); return q; };
    tb.logits = (float *)take(T * E * 4);
    tb.counts = (int32_t *)take(E * 4);
    tb.offsets = (int32_t *)take((E + 1) * 4);
    tb.active = (int32_t *)take(E * 4);
    tb.n_active = (int32_t *)take(4);
    tb.perm = (int32_t *)take(N * 4);
    tb.pos = (int32_t *)take(N * 4);
    tb.act = (float *)take(N * I * 4);
    tb.ysl = (float *)take(N * H * 4);
    return tb;
}

template <int T, bool GATE_UP>
static void launch_grouped_t(const localai_qmat *m, int lpr, int waves, const MoeTables &tb, const float *xsrc,
                             int64_t x_stride, int k, int slots, hipStream_t s) {
    const lq_geom &g = m->g;
    const int64_t half = GATE_UP ? g.rows / 2 : g.rows;
    const int64_t tile = MOE_R * (64 / lpr);
    dim3 grid((unsigned)((half + tile - 1) / tile), slots), block(64 * waves);
    const size_t lds = (size_t)waves * 2 * 16 * lpr * 16;
    if (lpr == 16)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 16>), grid, block, lds, s, m->data, g, tb, xsrc, x_stride, k);
    else if (lpr == 32)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 32>), grid, block, lds, s, m->data, g, tb, xsrc, x_stride, k);
    else
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 64>), grid, block, lds, s, m->data, g, tb, xsrc, x_stride, k);
}

template <bool GATE_UP>
static int launch_grouped(const localai_qmat *m, const MoeTables &tb, const float *xsrc, int64_t x_stride,
                          int k, int slots, hipStream_t s) {
    const lq_geom &g = m->g;
    const int lpr = lanes_per_row(g.nu);
    const int waves = lpr < 64 ? 1 : (int)((g.nu + 63) / 64);
    if (waves > 4) return fail(LOCALAI_EARG, "moe: expert K too large (more than 16384 values per row)");
    if ((size_t)waves * 2 * 16 * lpr * 16 > max_lds_per_block())
        return fail(LOCALAI_EARG, "moe: x windows exceed the LDS per workgroup");
    switch (g.type) {
#define LQ_G(TT) case TT: launch_grouped_t<TT, GATE_UP>(m, lpr, waves, tb, xsrc, x_stride, k, slots, s); break;
        LQ_G(LQ_Q4_K) LQ_G(LQ_Q5_K) LQ_G(LQ_Q6_K) LQ_G(LQ_Q8_0) LQ_G(LQ_Q4_0)
#undef LQ_G
        default: return fail(LOCALAI_ETYPE, "moe: unsupported expert type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_moe(const float *h, int64_t T, int64_t H, const float *rw, const float *rb, int64_t E, int k,
               const localai_qmat *gu, const localai_qmat *dn, float *out, int32_t *topk_idx, float *topk_w,
               void *ws, hipStream_t s) {
    const int64_t I = gu->g.rows / 2;
    MoeTables tb = carve(ws, T, E, k, H, I);
    size_t sh = (size_t)E * 4;
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)T), dim3(256), sh, s, h, (int)H, rw, rb, (int)E, k,
                       tb.logits, topk_idx, topk_w);
    LQ_HIP(hipGetLastError());
    size_t sh2 = (size_t)(34 * E + 1) * 4;
    hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(1024), sh2, s, topk_idx, (int)(T * k), (int)E, tb);
    LQ_HIP(hipGetLastError());
    const int slots = (int)(E < T * k ? E : T * k);
    if (int st = launch_grouped<true>(gu, tb, h, H, k, slots, s)) return st;
    if (int st = launch_grouped<false>(dn, tb, tb.act, I, k, slots, s)) return st;
    dim3 grid((unsigned)((H + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, s, tb.ysl, tb.pos, topk_w, k, (int)H, out);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
