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
//   route     one workgroup per token: router logits, top-k, gates (for a
//             single token also the permutation tables below)
//   permute   one workgroup: expert histogram, exclusive scan, stable
//             expert-major permutation of the T*k assignments (LDS)
//   gate_up   grouped matvec over the active experts, one workgroup per
//             (64-row gate tile + matching up tile, expert); SiLU*up fused
//   down      grouped matvec over the active experts
//   combine   gate-weighted sum of each token's k expert outputs (fixed order)
//
// Router logits are bit-reproducible: each is a sum of exact fp64 products
// h*w in a fixed order (lane l sums elements 256j + 4l + c, j-major; then a
// pairwise tree over the 64 lanes), rounded to fp32 once.
#include <math.h>

#include "gemv_core.h"
#include "internal.h"
#include "mfma_core.h"

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
    // prefill (expert GEMM) path
    int32_t *tile_e;    // [max_tiles] expert of each token tile
    int32_t *tile_p0;   // [max_tiles] first perm position of the tile
    int32_t *tile_n;    // [max_tiles] tokens in the tile (<= tile width)
    int32_t *n_tiles;   // [1]
    _Float16 *xh_gu;    // [N, ldh(H)] f16 token rows of h in perm order
    float *inv_gu;      // [N]
    _Float16 *xh_dn;    // [N, ldh(I)] f16 act rows
    float *inv_dn;      // [N]
    int max_tiles;
    int tile_w;         // tokens per tile (0: matvec path, no tile list)
};

// ------------------------------------------------------------------ route

// (logit desc, index asc); a NaN logit ranks below every number, NaNs by
// index -- the order of np.lexsort((index, -logit)) (oracle/moe.py topk)
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
    const bool na = va != va, nb = vb != vb;
    if (na || nb) return nb && (!na || ia < ib);
    return va > vb || (va == vb && ia < ib);
}

// Widest hidden size whose fp64 copy of h is staged in LDS (64 KiB); wider
// rows convert h in registers in every wave.
constexpr int ROUTE_LDS_H = 8192;

// One workgroup per token. h is converted to fp64 once (in LDS) and shared by
// the waves, each of which computes whole expert logits; wave 0 then ranks
// the experts. With `tables` (a single token) the workgroup also writes the
// expert-major permutation tables of moe_permute_kernel for its k
// assignments, so the layer needs no permute launch.
// LDS: E logits, k selected experts (8-byte aligned), then h as fp64.
template <bool LDS_H>
__global__ __launch_bounds__(1024) void moe_route_kernel(const float *__restrict__ h, int H,
                                                         const float *__restrict__ rw,
                                                         const float *__restrict__ rb, int E, int k,
                                                         float *__restrict__ logits,
                                                         int32_t *__restrict__ topk_idx,
                                                         float *__restrict__ topk_w, MoeTables tb, int tables) {
    extern __shared__ __attribute__((aligned(16))) float lg[];
    int *sel = reinterpret_cast<int *>(lg + E);
    double *h64 = reinterpret_cast<double *>(lg + ((E + k + 3) & ~3));
    const int t = blockIdx.x;
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    const float *ht = h + (int64_t)t * H;
    constexpr bool lds_h = LDS_H;   // H <= ROUTE_LDS_H
    if (lds_h) {
        for (int i = threadIdx.x * 4; i < H; i += blockDim.x * 4) {
            const float4 v = *reinterpret_cast<const float4 *>(ht + i);
            *reinterpret_cast<double2 *>(h64 + i) = make_double2(v.x, v.y);
            *reinterpret_cast<double2 *>(h64 + i + 2) = make_double2(v.z, v.w);
        }
        __syncthreads();
    }
    constexpr int CH = 8;                  // 16-byte chunks per lane loaded ahead of the sums
    for (int e = w; e < E; e += nw) {
        const float *we = rw + (int64_t)e * H;
        double s = 0.0;
        // lane l sums elements 256j + 4l + c (j = 0, 1, ..., c = 0..3) in that
        // order (exact fp64 products); H is a multiple of 4, so a chunk is
        // either wholly inside the row or wholly past its end
        for (int i0 = 0; i0 < H; i0 += 256 * CH) {
            float4 hv[CH], wv[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int i = i0 + 256 * j + 4 * lane;
                const int ic = i < H ? i : H - 4;      // unconditional loads: no wait per load
                wv[j] = *reinterpret_cast<const float4 *>(we + ic);
                if (!lds_h) hv[j] = *reinterpret_cast<const float4 *>(ht + ic);
            }
            __builtin_amdgcn_sched_barrier(0);   // every load issued before the first sum
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int i = i0 + 256 * j + 4 * lane;
                const bool in = i < H;           // chunks past H add exact zero products
                double2 a, b;
                if (lds_h) {
                    const int ic = in ? i : 0;
                    a = *reinterpret_cast<const double2 *>(h64 + ic);
                    b = *reinterpret_cast<const double2 *>(h64 + ic + 2);
                } else {
                    a = make_double2(hv[j].x, hv[j].y);
                    b = make_double2(hv[j].z, hv[j].w);
                }
                s = __builtin_fma(in ? a.x : 0.0, (double)wv[j].x, s);
                s = __builtin_fma(in ? a.y : 0.0, (double)wv[j].y, s);
                s = __builtin_fma(in ? b.x : 0.0, (double)wv[j].z, s);
                s = __builtin_fma(in ? b.y : 0.0, (double)wv[j].w, s);
            }
        }
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
    float myv = -INFINITY;
    int myi = 0;
    if (E <= 64) {
        // lane e ranks expert e against all E (values broadcast with
        // readlane): rank = number of experts that beat it; the rank-r expert
        // is choice r
        const float v = lane < E ? lg[lane] : 0.0f;
        int rank = 0;
        for (int j = 0; j < E; ++j)
            rank += better(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j)), j,
                           v, lane);
        if (lane < E && rank < k) sel[rank] = lane;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane < k) {
            myi = sel[lane];
            myv = lg[myi];
        }
    } else {
        // lane l owns experts l, l+64, ...; bit j of `taken` marks expert l+64j as selected
        uint32_t taken = 0;
        for (int r = 0; r < k; ++r) {
            float bv = __builtin_nanf("");   // ranks below every expert
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
    }
    // gates: softmax over the k selected logits, normaliser summed in choice order
    const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, myv), 0));
    const float ex = lane < k ? expf(myv - vmax) : 0.0f;
    float z = 0.0f;
    for (int j = 0; j < k; ++j) z += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), j));
    if (lane < k) {
        topk_idx[(int64_t)t * k + lane] = myi;
        topk_w[(int64_t)t * k + lane] = ex / z;
    }
    if (!tables) return;
    // one token: assignment a = lane (< k) has the distinct expert myi; its
    // position in expert-major order is the number of selected experts below it
    int rank = 0;
    for (int j = 0; j < k; ++j) rank += lane < k && __builtin_amdgcn_readlane(myi, j) < myi;
    if (lane < k) {
        tb.perm[rank] = lane;
        tb.pos[lane] = rank;
        tb.active[rank] = myi;
    }
    for (int e = lane; e <= E; e += 64) {
        int below = 0, hit = 0;
        for (int j = 0; j < k; ++j) {
            const int ej = __builtin_amdgcn_readlane(myi, j);
            below += ej < e;
            hit |= ej == e;
        }
        tb.offsets[e] = below;
        if (e < E) tb.counts[e] = hit;
    }
    if (lane == 0) tb.n_active[0] = k;
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
        int o = 0, na = 0, nt = 0;
        for (int e = 0; e < E; ++e) {
            off[e] = o;
            tb.offsets[e] = o;
            tb.counts[e] = total[e];
            if (total[e] > 0) tb.active[na++] = e;
            if (tb.tile_w > 0)
                for (int p = 0; p < total[e]; p += tb.tile_w) {
                    tb.tile_e[nt] = e;
                    tb.tile_p0[nt] = o + p;
                    tb.tile_n[nt] = min(tb.tile_w, total[e] - p);
                    ++nt;
                }
            o += total[e];
        }
        off[E] = o;
        tb.offsets[E] = o;
        tb.n_active[0] = na;
        if (tb.tile_w > 0) tb.n_tiles[0] = nt;
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

// register rows per lane: as the dense matvec (gemv.hip); split evenly
// between the gate and up halves for gate_up
template <int T, int NT>
constexpr int moe_rows() {
    return NT == 2 ? 4 : (T == LQ_Q6_K || T == LQ_Q5_K) ? 4 : 8;
}

// One workgroup: a tile of RS * G rows (RS register rows per row set, G =
// 64 / LPR lane groups) of one active expert, for NT of its tokens
// (blockIdx.z picks which). gate_up: rows r of the gate half and r + inter
// of the up half share the x staging and the reduction, and the output is
// silu(g) * u; down: rows r of the down matrix. With LPR = 64 the waves split
// the K units. A token pair whose second token does not exist repeats the
// first and skips its writes.
template <int T, bool GATE_UP, int LPR, int NT>
__global__ __launch_bounds__(256) void moe_grouped_kernel(const uint8_t *__restrict__ Wall, lq_geom g,
                                                          MoeTables tb, const float *__restrict__ xsrc,
                                                          int64_t x_stride, int k) {
    constexpr int R = moe_rows<T, NT>();
    constexpr int SETS = GATE_UP ? 2 : 1;
    constexpr int RS = R / SETS;
    constexpr int G = 64 / LPR;
    extern __shared__ float4 xlds[];             // NT * 16 * LPR float4 per wave
    __shared__ float red[4 * G * R * NT];        // [waves x groups][register rows][NT]
    const int slot = blockIdx.y;
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int n = tb.counts[e], base = tb.offsets[e];
    const int t0 = blockIdx.z * NT;
    if (t0 >= n) return;
    const int nv = n - t0 < NT ? n - t0 : NT;
    const uint8_t *Wexp = Wall + (int64_t)e * g.matrix_bytes;
    const int64_t half = GATE_UP ? g.rows / 2 : g.rows;
    const int64_t row0 = (int64_t)blockIdx.x * RS * G;
    // gate_up: x = token rows of h, out = act rows [p, inter]; down: x = act rows, out = ysl rows [p, H]
    const float *xrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int p = base + t0 + (t < nv ? t : 0);
        const int64_t src = GATE_UP ? (int64_t)(tb.perm[p] / k) : (int64_t)p;
        xrow[t] = xsrc + src * x_stride;
    }
    const int64_t out_stride = GATE_UP ? g.rows / 2 : g.rows;
    float *outp = (GATE_UP ? tb.act : tb.ysl) + (int64_t)(base + t0) * out_stride;
    const int w = wave_id(), nw = blockDim.x >> 6;
    int vi;
    bool writer;
    const float v = wave_rows<T, NT, 1, R, LPR, SETS>(Wexp, g, row0, half + row0, GATE_UP ? g.rows : half, w,
                                                      xrow, xlds + w * NT * 16 * LPR, vi, writer);
    // value r * NT + t; the up-half rows (set 1) follow the RS * NT set-0 values
    if (writer) red[(w * G + lane_id() / LPR) * R * NT + vi] = v;
    __syncthreads();
    const int i = threadIdx.x;
    if (i < G * RS * NT) {
        const int gi = i / (RS * NT), j = i % (RS * NT);
        float sa = 0.0f, sb = 0.0f;
        for (int kk = 0; kk < nw; ++kk) {
            sa += red[(kk * G + gi) * R * NT + j];
            if (GATE_UP) sb += red[(kk * G + gi) * R * NT + RS * NT + j];
        }
        const int r = j / NT, t = j % NT;
        const int64_t row = row0 + gi * RS + r;
        if (t < nv && row < half) outp[t * out_stride + row] = GATE_UP ? silu(sa) * sb : sa;
    }
}

// -------------------------------------------- grouped matvec on i8 MFMA
// Decode path for expert tensors that have the tile form (Q4_K / Q6_K,
// mfma_core.h). A workgroup loads its weight tiles once and walks the tokens
// routed to its expert, restaging x per token.

// gate_up: workgroup (i, slot) = gate tile i (rows 16i ..) and up tile
// inter / 16 + i of the slot's expert; act[p, 16i + n] = silu(g) * u
// (engine/zaya.py:303-306) for every perm position p of the expert.
// `single` (one token): slot = assignment a, expert topk_idx[a], act row a --
// the weights are requested after one dependent load.
template <int TYPE, int SPW, int MAXT>
__global__ __launch_bounds__(MAXT) void moe_mfma_gate_up(const uint8_t *__restrict__ Wt, int64_t mat_bytes, int nb,
                                                         int64_t inter, MoeTables tb, const float *__restrict__ h,
                                                         int64_t H, int k, const int32_t *__restrict__ topk_idx,
                                                         int single, float *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    int e;
    if (single) {
        e = topk_idx[slot];
        if (slot == 0) {   // clear the token's output for moe_mfma_down_single
            const int64_t per = (H + gridDim.x - 1) / gridDim.x;
            for (int64_t c = blockIdx.x * per + threadIdx.x; c < (blockIdx.x + 1) * per && c < H; c += blockDim.x)
                out[c] = 0.0f;
        }
    } else {
        if (slot >= tb.n_active[0]) return;
        e = tb.active[slot];
    }
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x, tile_bytes = (int64_t)nb * mt_block_bytes(TYPE);
    const uint8_t *We = Wt + (int64_t)e * mat_bytes;
    MtW<TYPE> w[2][SPW];
    mt_load_tile<TYPE, SPW>(w[0], We + i * tile_bytes, nb, sb0, nsb, lane);
    mt_load_tile<TYPE, SPW>(w[1], We + (inter / MT_ROWS + i) * tile_bytes, nb, sb0, nsb, lane);
    __builtin_amdgcn_sched_barrier(0);
    // the expert's tokens; each next token's row is requested before the
    // current token's arithmetic
    const int n = single ? 1 : tb.counts[e], base = single ? slot : tb.offsets[e];
    const int tok0 = single ? 0 : tb.perm[base] / k;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], h + (int64_t)tok0 * H, nb, sb0, lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xn[1][SPW];
        if (j + 1 < n) mt_load_x<SPW>(xn[0], h + (int64_t)(tb.perm[p + 1] / k) * H, nb, sb0, lane);
        float *fin;
        mt_pass<TYPE, SPW, 2, 1>(w, xv, nsb, smem, fin);
        const int r = threadIdx.x;
        if (r < MT_ROWS) tb.act[(int64_t)p * inter + i * MT_ROWS + r] = silu(fin[r]) * fin[MT_ROWS + r];
        if (j + 1 < n) {
#pragma unroll
            for (int kk = 0; kk < SPW; ++kk) xv[0][kk] = xn[0][kk];
        }
    }
}

// down: workgroup (i, slot) = hidden tile i of the slot's expert;
// ysl[p, 16i + n] for every perm position p of the expert
template <int TYPE, int SPW, int MAXT>
__global__ __launch_bounds__(MAXT) void moe_mfma_down(const uint8_t *__restrict__ Wt, int64_t mat_bytes, int nb,
                                                      int64_t hidden, MoeTables tb, int64_t inter) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int n = tb.counts[e], base = tb.offsets[e];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], tb.act + (int64_t)base * inter, nb, sb0, lane);
    MtW<TYPE> w[1][SPW];
    mt_load_tile<TYPE, SPW>(w[0], Wt + (int64_t)e * mat_bytes + i * nb * mt_block_bytes(TYPE), nb, sb0, nsb, lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xn[1][SPW];
        if (j + 1 < n) mt_load_x<SPW>(xn[0], tb.act + (int64_t)(p + 1) * inter, nb, sb0, lane);
        float *fin;
        mt_pass<TYPE, SPW, 1, 1>(w, xv, nsb, smem, fin);
        const int r = threadIdx.x;
        if (r < MT_ROWS && i * MT_ROWS + r < hidden) tb.ysl[(int64_t)p * hidden + i * MT_ROWS + r] = fin[r];
        if (j + 1 < n) {
#pragma unroll
            for (int kk = 0; kk < SPW; ++kk) xv[0][kk] = xn[0][kk];
        }
    }
}

// One token (decode), k <= 2: workgroup (i, s) = hidden tile i of expert
// topk_idx[s]; out[16i + n] += topk_w[s] * y (out cleared by gate_up). Two
// additions onto zero give the same sum in either order, so the result does
// not depend on which workgroup lands first.
template <int TYPE, int SPW, int MAXT>
__global__ __launch_bounds__(MAXT) void moe_mfma_down_single(const uint8_t *__restrict__ Wt, int64_t mat_bytes,
                                                             int nb, int64_t hidden, MoeTables tb, int64_t inter,
                                                             const int32_t *__restrict__ topk_idx,
                                                             const float *__restrict__ topk_w,
                                                             float *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x;
    const int s = blockIdx.y;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], tb.act + (int64_t)s * inter, nb, sb0, lane);
    MtW<TYPE> w[1][SPW];
    mt_load_tile<TYPE, SPW>(w[0], Wt + (int64_t)topk_idx[s] * mat_bytes + i * nb * mt_block_bytes(TYPE), nb, sb0,
                            nsb, lane);
    __builtin_amdgcn_sched_barrier(0);
    float *fin;
    mt_pass<TYPE, SPW, 1, 1>(w, xv, nsb, smem, fin);
    const int r = threadIdx.x;
    if (r < MT_ROWS && i * MT_ROWS + r < hidden) atomicAdd(out + i * MT_ROWS + r, topk_w[s] * fin[r]);
}

// One token (decode): hidden tile i of each of its K experts, with the gate
// weighted sum of moe_combine_kernel in the epilogue (same order, same fma
// chain, so the result equals down + combine). act rows are in assignment
// order (gate_up `single`).
template <int TYPE, int SPW, int K, int MAXT>
__global__ __launch_bounds__(MAXT) void moe_mfma_down_combine(const uint8_t *__restrict__ Wt, int64_t mat_bytes,
                                                              int nb, int64_t hidden, MoeTables tb, int64_t inter,
                                                              const int32_t *__restrict__ topk_idx,
                                                              const float *__restrict__ topk_w,
                                                              float *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x;
    float4 xv[K][SPW];
    MtW<TYPE> w[K][SPW];
#pragma unroll
    for (int s = 0; s < K; ++s) mt_load_x<SPW>(xv[s], tb.act + (int64_t)s * inter, nb, sb0, lane);
#pragma unroll
    for (int s = 0; s < K; ++s)
        mt_load_tile<TYPE, SPW>(w[s], Wt + (int64_t)topk_idx[s] * mat_bytes + i * nb * mt_block_bytes(TYPE), nb,
                                sb0, nsb, lane);
    __builtin_amdgcn_sched_barrier(0);
    float *fin;
    mt_pass<TYPE, SPW, K, K>(w, xv, nsb, smem, fin);
    const int r = threadIdx.x;
    if (r < MT_ROWS && i * MT_ROWS + r < hidden) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < K; ++s) acc = __builtin_fmaf(topk_w[s], fin[s * MT_ROWS + r], acc);
        out[i * MT_ROWS + r] = acc;
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

// Tokens at or above which the layer runs the expert GEMM path (prefill).
constexpr int64_t MOE_GEMM_TOKENS = 32;

static int64_t moe_max_tiles(int64_t N, int64_t E, int tile_w) {
    return N / tile_w + (E < N ? E : N);
}

// f16 token rows, zero-padded to a multiple of 256 values (gemm.hip)
static int64_t f16_stride(int64_t cols) { return 256 * ((cols + 255) / 256); }

size_t moe_workspace_bytes(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const int64_t N = T * k;
    size_t s = 0;
    s += align256(T * E * 4);                                        // logits
    s += align256(E * 4) * 2 + align256((E + 1) * 4) + align256(4);  // counts, offsets, active, n_active
    s += align256(N * 4) * 2;                                        // perm, pos
    s += align256(N * I * 4);                                        // act
    s += align256(N * H * 4);                                        // ysl
    if (T >= MOE_GEMM_TOKENS) {
        const int64_t mt = moe_max_tiles(N, E, moe_gemm_tile());
        s += align256(mt * 4) * 3 + align256(4);
        s += align256(N * f16_stride(H) * 2) + align256(N * 4);
        s += align256(N * f16_stride(I) * 2) + align256(N * 4);
    }
    return s;
}

static MoeTables carve(void *ws, int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const int64_t N = T * k;
    uint8_t *p = (uint8_t *)ws;
    MoeTables tb{};
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
    tb.tile_w = 0;
    if (T >= MOE_GEMM_TOKENS) {
        tb.tile_w = moe_gemm_tile();
        tb.max_tiles = (int)moe_max_tiles(N, E, tb.tile_w);
        tb.tile_e = (int32_t *)take(tb.max_tiles * 4);
        tb.tile_p0 = (int32_t *)take(tb.max_tiles * 4);
        tb.tile_n = (int32_t *)take(tb.max_tiles * 4);
        tb.n_tiles = (int32_t *)take(4);
        tb.xh_gu = (_Float16 *)take(N * f16_stride(H) * 2);
        tb.inv_gu = (float *)take(N * 4);
        tb.xh_dn = (_Float16 *)take(N * f16_stride(I) * 2);
        tb.inv_dn = (float *)take(N * 4);
    }
    return tb;
}

template <int T, bool GATE_UP, int NT>
static void launch_grouped_t(const localai_qmat *m, int lpr, int waves, const MoeTables &tb, const float *xsrc,
                             int64_t x_stride, int k, int slots, int64_t max_tokens, hipStream_t s) {
    const lq_geom &g = m->g;
    const int64_t half = GATE_UP ? g.rows / 2 : g.rows;
    const int64_t tile = (int64_t)(moe_rows<T, NT>() / (GATE_UP ? 2 : 1)) * (64 / lpr);
    dim3 grid((unsigned)((half + tile - 1) / tile), slots, (unsigned)((max_tokens + NT - 1) / NT)),
        block(64 * waves);
    const size_t lds = (size_t)waves * NT * 16 * lpr * 16;
    if (lpr == 16)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 16, NT>), grid, block, lds, s, m->data, g, tb, xsrc,
                           x_stride, k);
    else if (lpr == 32)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 32, NT>), grid, block, lds, s, m->data, g, tb, xsrc,
                           x_stride, k);
    else
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 64, NT>), grid, block, lds, s, m->data, g, tb, xsrc,
                           x_stride, k);
}

// max_tokens: an upper bound on the tokens routed to one expert (the token
// count); workgroups past an expert's count exit at once.
template <bool GATE_UP>
static int launch_grouped(const localai_qmat *m, const MoeTables &tb, const float *xsrc, int64_t x_stride,
                          int k, int slots, int64_t max_tokens, hipStream_t s) {
    const lq_geom &g = m->g;
    const int lpr = lanes_per_row(g.nu);
    const int waves = lpr < 64 ? 1 : (int)((g.nu + 63) / 64);
    const int nt = max_tokens >= 2 ? 2 : 1;
    if (waves > 4) return fail(LOCALAI_EARG, "moe: expert K too large (more than 16384 values per row)");
    if ((size_t)waves * nt * 16 * lpr * 16 > max_lds_per_block())
        return fail(LOCALAI_EARG, "moe: x windows exceed the LDS per workgroup");
    if ((max_tokens + nt - 1) / nt > 65535) return fail(LOCALAI_EARG, "moe: too many tokens for the matvec path");
    switch (g.type) {
#define LQ_G(TT)                                                                                      \
    case TT:                                                                                          \
        if (nt == 2) launch_grouped_t<TT, GATE_UP, 2>(m, lpr, waves, tb, xsrc, x_stride, k, slots, max_tokens, s); \
        else launch_grouped_t<TT, GATE_UP, 1>(m, lpr, waves, tb, xsrc, x_stride, k, slots, max_tokens, s);        \
        break;
        LQ_G(LQ_Q4_K) LQ_G(LQ_Q5_K) LQ_G(LQ_Q6_K) LQ_G(LQ_Q8_0) LQ_G(LQ_Q4_0)
#undef LQ_G
        default: return fail(LOCALAI_ETYPE, "moe: unsupported expert type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// MFMA decode path: both expert tensors in the tile form with K <= 32
// super-blocks: one super-block per wave (up to 16 waves) for K <= 16
// super-blocks, else four per wave (up to 8 waves, room for the registers).
static bool moe_mfma_ok(const localai_qmat *gu, const localai_qmat *dn, const float *h, int64_t H, int64_t I) {
    return gu->tiles && dn->tiles && gu->g.type == dn->g.type && gu->g.type != LQ_Q8_0 && gu->g.nb <= 32 &&
           dn->g.nb <= 32 &&
           (reinterpret_cast<uintptr_t>(h) & 15) == 0 && I % MT_ROWS == 0 && gu->g.cols == H && dn->g.cols == I;
}

template <int TYPE>
static int launch_moe_mfma_t(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                             int64_t T, int64_t H, int64_t I, int k, int slots, const int32_t *topk_idx,
                             const float *topk_w, float *out, bool fused_combine, hipStream_t s) {
    {
        const int nb = (int)gu->g.nb, spw = nb <= 16 ? 1 : 4, waves = (nb + spw - 1) / spw;
        dim3 grid((unsigned)(I / MT_ROWS), slots), block(64 * waves);
        const size_t lds = mt_lds_bytes(TYPE, waves, spw, 1, 2);
        const int single = fused_combine;   // one token: assignment-ordered act rows
        if (spw == 1)
            hipLaunchKernelGGL((moe_mfma_gate_up<TYPE, 1, 1024>), grid, block, lds, s, gu->tiles, gu->tile_bytes, nb,
                               I, tb, h, H, k, topk_idx, single, out);
        else
            hipLaunchKernelGGL((moe_mfma_gate_up<TYPE, 4, 512>), grid, block, lds, s, gu->tiles, gu->tile_bytes, nb,
                               I, tb, h, H, k, topk_idx, single, out);
        LQ_HIP(hipGetLastError());
    }
    const int nb = (int)dn->g.nb, spw = nb <= 16 ? 1 : 4, waves = (nb + spw - 1) / spw;
    const unsigned tiles = (unsigned)((H + MT_ROWS - 1) / MT_ROWS);
    if (fused_combine) {
        const size_t lds = mt_lds_bytes(TYPE, waves, spw, 1, 1);
        if (spw == 1)
            hipLaunchKernelGGL((moe_mfma_down_single<TYPE, 1, 1024>), dim3(tiles, k), dim3(64 * waves), lds, s,
                               dn->tiles, dn->tile_bytes, nb, H, tb, I, topk_idx, topk_w, out);
        else
            hipLaunchKernelGGL((moe_mfma_down_single<TYPE, 4, 512>), dim3(tiles, k), dim3(64 * waves), lds, s,
                               dn->tiles, dn->tile_bytes, nb, H, tb, I, topk_idx, topk_w, out);
    } else {
        const size_t lds = mt_lds_bytes(TYPE, waves, spw, 1, 1);
        if (spw == 1)
            hipLaunchKernelGGL((moe_mfma_down<TYPE, 1, 1024>), dim3(tiles, slots), dim3(64 * waves), lds, s,
                               dn->tiles, dn->tile_bytes, nb, H, tb, I);
        else
            hipLaunchKernelGGL((moe_mfma_down<TYPE, 4, 512>), dim3(tiles, slots), dim3(64 * waves), lds, s,
                               dn->tiles, dn->tile_bytes, nb, H, tb, I);
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_moe(const float *h, int64_t T, int64_t H, const float *rw, const float *rb, int64_t E, int k,
               const localai_qmat *gu, const localai_qmat *dn, float *out, int32_t *topk_idx, float *topk_w,
               void *ws, hipStream_t s) {
    const int64_t I = gu->g.rows / 2;
    MoeTables tb = carve(ws, T, E, k, H, I);
    const int64_t hpad = H <= ROUTE_LDS_H ? H : 0;   // fp64 copy of h in LDS
    size_t sh = (size_t)((E + k + 3) & ~3) * 4 + (size_t)hpad * 8;
    const int one = T == 1 && tb.tile_w == 0;   // single token: the router writes the tables
    if (hpad)
        hipLaunchKernelGGL(moe_route_kernel<true>, dim3((unsigned)T), dim3(1024), sh, s, h, (int)H, rw, rb, (int)E, k,
                           tb.logits, topk_idx, topk_w, tb, one);
    else
        hipLaunchKernelGGL(moe_route_kernel<false>, dim3((unsigned)T), dim3(1024), sh, s, h, (int)H, rw, rb, (int)E,
                           k, tb.logits, topk_idx, topk_w, tb, one);
    LQ_HIP(hipGetLastError());
    if (!one) {
        size_t sh2 = (size_t)(34 * E + 1) * 4;
        hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(1024), sh2, s, topk_idx, (int)(T * k), (int)E, tb);
        LQ_HIP(hipGetLastError());
    }
    const int slots = (int)(E < T * k ? E : T * k);
    if (tb.tile_w > 0) {
        // prefill: gathered f16 token rows -> expert GEMMs on MFMA
        const int64_t N = T * k;
        if (gu->g.cols != H || dn->g.cols != I) return fail(LOCALAI_EARG, "moe: expert shapes");
        if (int st = launch_x_to_f16(h, H, H, tb.perm, k, N, tb.xh_gu, f16_stride(H), tb.inv_gu, s)) return st;
        if (int st = launch_moe_gemm(gu->g, gu->data, gu->tiles, gu->tile_bytes, true, tb.xh_gu, f16_stride(H),
                                     tb.inv_gu, tb.act, I, I,
                                     tb.tile_e, tb.tile_p0, tb.tile_n, tb.n_tiles, tb.max_tiles, s))
            return st;
        if (int st = launch_x_to_f16(tb.act, I, I, nullptr, 1, N, tb.xh_dn, f16_stride(I), tb.inv_dn, s)) return st;
        if (int st = launch_moe_gemm(dn->g, dn->data, dn->tiles, dn->tile_bytes, false, tb.xh_dn, f16_stride(I),
                                     tb.inv_dn, tb.ysl, H, I,
                                     tb.tile_e, tb.tile_p0, tb.tile_n, tb.n_tiles, tb.max_tiles, s))
            return st;
    } else if (moe_mfma_ok(gu, dn, h, H, I)) {
        // decode on MFMA; one token with k <= 2 folds the combine into down
        const bool fused = T == 1 && k <= 2;
        const int st = gu->g.type == LQ_Q6_K
                           ? launch_moe_mfma_t<LQ_Q6_K>(gu, dn, tb, h, T, H, I, k, slots, topk_idx, topk_w, out, fused, s)
                           : launch_moe_mfma_t<LQ_Q4_K>(gu, dn, tb, h, T, H, I, k, slots, topk_idx, topk_w, out, fused, s);
        if (st || fused) return st;
    } else {
        if (int st = launch_grouped<true>(gu, tb, h, H, k, slots, T, s)) return st;
        if (int st = launch_grouped<false>(dn, tb, tb.act, I, k, slots, T, s)) return st;
    }
    dim3 grid((unsigned)((H + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, s, tb.ysl, tb.pos, topk_w, k, (int)H, out);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
