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
//   route     few tokens: the router logits, one one-wave workgroup per
//             (expert, token); many tokens: register-tiled logits over
//             LDS-streamed rows, then one wave per token for top-k and gates
//   permute   one workgroup (few tokens: first top-k and gates, one wave per
//             token): ballot-matched ranks per wave, per-expert scan, stable
//             expert-major permutation of the T*k assignments and the expert
//             GEMM tile list
//   gate_up   grouped matvec over the active experts, one workgroup per
//             (64-row gate tile + matching up tile, expert); SiLU*up fused
//   down      grouped matvec over the active experts
//   combine   gate-weighted sum of each token's k expert outputs (fixed order)
// One token with k <= 2 on MFMA: route, then gate_up and down in a single
// launch (moe_decode1_kernel: the down tiles' weights stream beside
// gate_up's, the combine folded into down). From 32 tokens: the expert
// GEMMs on MFMA (gemm.hip) between the permute and the combine.
//
// Router logits are bit-reproducible: each is a sum of exact fp64 products
// h*w in a fixed order (lane l sums elements 256j + 4l + c, j-major; then a
// pairwise tree over the 64 lanes), rounded to fp32 once.
#include <math.h>

#include <atomic>

#include "gemv_core.h"
#include "internal.h"
#include "f16rows.h"
#include "fused_sync.h"
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
    _Float16 *xh_gu;    // [T, ldh(H)] f16 token rows of h
    float *inv_gu;      // [T]
    float *hn2;         // [T] sum of squares of each token row of h
    _Float16 *xh_dn;    // [N, ldh(I)] f16 act rows
    float *inv_dn;      // [N]
    int max_tiles;
    int tile_w;         // tokens per tile (0: matvec path, no tile list)
    uint32_t *sync;     // counters of the fused one-token layer (1 KiB)
};

// ------------------------------------------------------------------ route

// Expert order: (logit desc, index asc); a NaN logit ranks below every
// number, NaNs by index -- the order of np.lexsort((index, -logit))
// (oracle/moe.py topk). route_key maps a logit to an unsigned key with the
// same order on values: numbers by their IEEE order (-0 and +0 equal) from
// 0x007fffff up, NaN 1; 0 is left for experts out of the running.
__device__ __forceinline__ uint32_t route_key(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t m = b == 0x80000000u ? 0x80000000u : (b & 0x80000000u ? ~b : b | 0x80000000u);
    return v != v ? 1u : m;
}

// Expert selection for token t by one whole wave from its E logits lg (LDS
// or global): top-k in expert order, gates = softmax over the k selected
// logits (normaliser summed in choice order), written to topk_idx / topk_w.
// Lane l holds the keys of experts l + 64 j; each of the k rounds takes the
// wave's largest key, the lowest index among the experts holding it, and
// drops that expert from the running. With `tables` (a single token) the
// wave also writes the expert-major permutation tables of moe_permute_kernel
// for the token's k assignments.
// MJ >= (E + 63) / 64: expert slots per lane.
template <int MJ>
__device__ __forceinline__ void route_select(const float *lg, int E, int k, int t, int32_t *__restrict__ topk_idx,
                                             float *__restrict__ topk_w, const MoeTables &tb, int tables) {
    const int lane = lane_id();
    const int nj = (E + 63) >> 6;
    float v[MJ];
    uint32_t key[MJ];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int e = lane + 64 * j;
        v[j] = j < nj && e < E ? lg[e] : 0.0f;   // every load issued before the first key
    }
#pragma unroll
    for (int j = 0; j < MJ; ++j) key[j] = j < nj && lane + 64 * j < E ? route_key(v[j]) : 0u;
    int myi = 0;
    float myv = 0.0f;
    for (int r = 0; r < k; ++r) {
        // the lane's best: the largest key, the lower j on equal keys
        uint32_t lk = 0, lj = 0;
#pragma unroll
        for (int j = 0; j < MJ; ++j) {
            const bool up = j < nj && key[j] > lk;
            lk = up ? key[j] : lk;
            lj = up ? j : lj;
        }
        const uint32_t top = wave_max_u32(lk);
        const uint32_t bi = wave_min_u32(lk == top ? (uint32_t)lane + 64u * lj : 0xffffffffu);
        const int bj = (int)(bi >> 6);
        float bv = v[0];
#pragma unroll
        for (int j = 1; j < MJ; ++j) bv = j == bj ? v[j] : bv;
        bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bv), (int)(bi & 63)));
#pragma unroll
        for (int j = 0; j < MJ; ++j) key[j] = lane + 64 * j == (int)bi ? 0u : key[j];
        myi = lane == r ? (int)bi : myi;
        myv = lane == r ? bv : myv;
    }
    const float vmax = uniform_f(myv, 0);
    const float ex = lane < k ? expf(myv - vmax) : 0.0f;
    float z = 0.0f;
    for (int j = 0; j < k; ++j) z += uniform_f(ex, j);
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

__device__ __forceinline__ void route_select_any(const float *lg, int E, int k, int t, int32_t *__restrict__ topk_idx,
                                                 float *__restrict__ topk_w, const MoeTables &tb, int tables) {
    if (E <= 64)
        route_select<1>(lg, E, k, t, topk_idx, topk_w, tb, tables);
    else if (E <= 128)
        route_select<2>(lg, E, k, t, topk_idx, topk_w, tb, tables);
    else if (E <= 256)
        route_select<4>(lg, E, k, t, topk_idx, topk_w, tb, tables);
    else
        route_select<16>(lg, E, k, t, topk_idx, topk_w, tb, tables);
}

// From this many tokens on, the logits come from moe_route_logits_kernel and
// the selection from moe_topk_kernel; below, from moe_route1_kernel and the
// permutation.
constexpr int ROUTE_TILE_TOKENS = 16;
// 16-byte chunks per lane and pass of moe_route1_kernel: rows of up to 2048
// elements in one pass.
constexpr int ROUTE_CH = 8;

// Router logits of a few tokens spread over E x T one-wave workgroups:
// workgroup (e, t) computes logit e of token t as the canonical sum (lane l
// sums elements 256 j + 4 l + c in (j, c) order as exact fp64 products,
// chunks past H adding exact zero products, then the butterfly), rounded to
// fp32 once. One workgroup per token (each wave one expert row at a time)
// took 5.5 us at 8 tokens x 16 experts and 20 us for one token of 128
// experts; E x T workgroups read the rows at the same time. Workgroup
// (0, 0) also clears the counter block of moe_decode1_kernel, which then
// selects the experts itself (else the permutation selects them). PART: H
// is not a multiple of 256 * ROUTE_CH.
template <bool PART>
__global__ __launch_bounds__(64) void moe_route1_kernel(const float *__restrict__ h, int H,
                                                        const float *__restrict__ rw,
                                                        const float *__restrict__ rb, float *__restrict__ logits,
                                                        uint32_t *__restrict__ sync) {
    const int lane = threadIdx.x, e = blockIdx.x;
    if (e == 0 && blockIdx.y == 0)
        for (int i = lane; i < D1_WORDS; i += 64) sync[i] = 0u;
    h += (int64_t)blockIdx.y * H;
    logits += (int64_t)blockIdx.y * gridDim.x;
    constexpr int CH = ROUTE_CH;
    const float *row = rw + (int64_t)e * H;
    double s = 0.0;
    for (int i0 = 0; i0 < H; i0 += 256 * CH) {
        float4 wv[CH], hv[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int i = i0 + 256 * j + 4 * lane;
            const int ic = i < H ? i : H - 4;
            wv[j] = *reinterpret_cast<const float4 *>(row + ic);
            hv[j] = *reinterpret_cast<const float4 *>(h + ic);
        }
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const bool in = !PART || i0 + 256 * j + 4 * lane < H;
            s = __builtin_fma(in ? (double)hv[j].x : 0.0, (double)wv[j].x, s);
            s = __builtin_fma(in ? (double)hv[j].y : 0.0, (double)wv[j].y, s);
            s = __builtin_fma(in ? (double)hv[j].z : 0.0, (double)wv[j].z, s);
            s = __builtin_fma(in ? (double)hv[j].w : 0.0, (double)wv[j].w, s);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) {
        float f = (float)s;
        if (rb) f = f + rb[e];
        logits[e] = f;
    }
}

// Tile of the many-token router: each wave covers RL_T tokens x RL_E
// experts, a workgroup RL_WT x RL_WE such tiles, i.e. RL_TOK token rows and
// RL_EXP expert rows.
constexpr int RL_T = 4, RL_E = 8;
constexpr int RL_WT = 4, RL_WE = 2;
constexpr int RL_NW = RL_WT * RL_WE;        // waves per workgroup
constexpr int RL_TOK = RL_T * RL_WT, RL_EXP = RL_E * RL_WE;
constexpr int RL_ROWS = RL_TOK + RL_EXP;   // rows of a 256-element chunk, 1 KiB each
constexpr int RL_RPW = RL_ROWS / RL_NW;    // rows each wave copies per chunk
constexpr int RL_STAGES = 3;               // chunks in LDS: one summed, two in flight
constexpr int RL_PAIRS = 16;               // (token, expert) pairs reduced per LDS round
constexpr int RL_LD = 68;                  // LDS row of a pair: 64 lane partials + 4 doubles of bank skew
static_assert(RL_ROWS % RL_NW == 0 && RL_RPW == 4, "the chunk wait below counts 4 copies per wave");
static_assert(RL_NW * RL_PAIRS * RL_LD * 8 <= RL_STAGES * RL_ROWS * 1024, "reduction fits the chunk stages");

// Router logits for many tokens, equal bit for bit to moe_route1_kernel's:
// lane l of each wave accumulates, for each (token, expert) pair of its
// RL_T x RL_E tile, the exact fp64 products of elements 256 j + 4 l + c in
// (j, c) order. The workgroup's RL_ROWS rows stream through LDS one 256-
// element chunk at a time, copied straight from global memory
// (global_load_lds, no registers) two chunks ahead of the one being summed,
// so the HBM latency is covered without occupancy. Each element is converted
// to fp64 once per wave tile and used for RL_E (token) or RL_T (expert)
// products. The 64 lane partials of a pair then meet in LDS and are added in
// the tree order of the wave reduction (s[l] += s[l + off], off = 32, 16,
// ..., 1): lane q of a group of four adds the 16 partials of lanes q, q + 4,
// ... (offsets 32, 16, 8, 4), then the group's four sums are combined
// across lanes (offsets 2, 1). Logits go to logits[T, E] as fp32 plus the
// bias. PART: H is not a multiple of 256 (the last chunk is partial).
template <bool PART>
__global__ __launch_bounds__(64 * RL_NW) void moe_route_logits_kernel(const float *__restrict__ h, int T, int H,
                                                               const float *__restrict__ rw,
                                                               const float *__restrict__ rb, int E,
                                                               float *__restrict__ logits) {
    __shared__ __attribute__((aligned(16))) float4 stage[RL_STAGES][RL_ROWS][64];
    const int lane = lane_id(), w = wave_id();
    const int wt = w / RL_WE, we = w % RL_WE;
    const int tb = blockIdx.x * RL_TOK, eb = blockIdx.y * RL_EXP;
    // copies: wave w fills rows w, w + RL_NW, ...; rows past T or E repeat the last one
    const float *src[RL_RPW];
#pragma unroll
    for (int i = 0; i < RL_RPW; ++i) {
        const int r = w + RL_NW * i;
        src[i] = (r < RL_TOK ? h + (int64_t)min(tb + r, T - 1) * H : rw + (int64_t)min(eb + r - RL_TOK, E - 1) * H) +
                 4 * lane;
    }
    const int nch = (H + 255) >> 8;
    auto issue = [&](int j, int b) {
        const int off = j << 8;
        // lanes past the end of a partial chunk copy the row's last 16 bytes
        const int o = !PART || off + 4 * lane < H ? off : H - 4 - 4 * lane;
#pragma unroll
        for (int i = 0; i < RL_RPW; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(src[i] + o),
                                             (__attribute__((address_space(3))) void *)&stage[b][w + RL_NW * i][0], 16,
                                             0, 0);
    };
    double acc[RL_T][RL_E];
#pragma unroll
    for (int a = 0; a < RL_T; ++a)
#pragma unroll
        for (int b = 0; b < RL_E; ++b) acc[a][b] = 0.0;
    // chunk j sits in stage j % RL_STAGES; chunk j + 2 is requested while
    // chunk j is summed. Every wait is unconditional so that the build's
    // assembly check can prove it (isa_check.lds_ring_violations): the loop
    // runs while chunk j + 2 exists, then the last two chunks are peeled.
    auto sum_chunk = [&](int j, int b) {
        // the chunk's rows, read in one block that waits for its own results
        // (the compiler would otherwise wait for every copy in flight first);
        // early-clobber outputs keep the addresses alive through the block
        lq_f4 hv[RL_T], wv[RL_E];
        const uint32_t ah = (uint32_t)(uintptr_t)&stage[b][wt * RL_T][lane];
        const uint32_t aw = (uint32_t)(uintptr_t)&stage[b][RL_TOK + we * RL_E][lane];
        static_assert(RL_T == 4 && RL_E == 8, "the read block below names 4 token and 8 expert rows");
        asm volatile(
            "ds_read_b128 %0, %12\n"
            "ds_read_b128 %1, %12 offset:1024\n"
            "ds_read_b128 %2, %12 offset:2048\n"
            "ds_read_b128 %3, %12 offset:3072\n"
            "ds_read_b128 %4, %13\n"
            "ds_read_b128 %5, %13 offset:1024\n"
            "ds_read_b128 %6, %13 offset:2048\n"
            "ds_read_b128 %7, %13 offset:3072\n"
            "ds_read_b128 %8, %13 offset:4096\n"
            "ds_read_b128 %9, %13 offset:5120\n"
            "ds_read_b128 %10, %13 offset:6144\n"
            "ds_read_b128 %11, %13 offset:7168\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hv[0]), "=&v"(hv[1]), "=&v"(hv[2]), "=&v"(hv[3]), "=&v"(wv[0]), "=&v"(wv[1]),
              "=&v"(wv[2]), "=&v"(wv[3]), "=&v"(wv[4]), "=&v"(wv[5]), "=&v"(wv[6]), "=&v"(wv[7])
            : "v"(ah), "v"(aw)
            : "memory");
        if (PART && j == nch - 1 && (j << 8) + 4 * lane >= H) {
            // past the end of the row: exact zero products
            const lq_f4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < RL_T; ++i) hv[i] = z;
#pragma unroll
            for (int i = 0; i < RL_E; ++i) wv[i] = z;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            double hd[RL_T], wd[RL_E];
#pragma unroll
            for (int i = 0; i < RL_T; ++i) hd[i] = (double)hv[i][c];
#pragma unroll
            for (int i = 0; i < RL_E; ++i) wd[i] = (double)wv[i][c];
#pragma unroll
            for (int a = 0; a < RL_T; ++a)
#pragma unroll
                for (int e = 0; e < RL_E; ++e) acc[a][e] = __builtin_fma(hd[a], wd[e], acc[a][e]);
        }
    };
    issue(0, 0);
    if (nch > 1) issue(1, 1);
    int j = 0, b = 0;   // chunk j in stage b
    for (; j + 2 < nch; ++j) {
        // this wave's copies of chunk j are done once only chunk j + 1's remain
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        // every wave's copies of chunk j have landed, and every wave has read
        // chunk j - 1 (its reads completed before its sums), whose stage is
        // refilled next. A bare barrier: __syncthreads' fence would also wait
        // for the copies still in flight.
        asm volatile("s_barrier" ::: "memory");
        issue(j + 2, b == 0 ? 2 : b - 1);
        sum_chunk(j, b);
        b = b == RL_STAGES - 1 ? 0 : b + 1;
    }
    if (j + 1 < nch) {   // chunk nch - 2: only chunk nch - 1's copies may remain
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        sum_chunk(j, b);
        b = b == RL_STAGES - 1 ? 0 : b + 1;
        ++j;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the last chunk
    asm volatile("s_barrier" ::: "memory");
    sum_chunk(j, b);
    __syncthreads();   // the stages become the reduction buffer
    double *rd = reinterpret_cast<double *>(&stage[0][0][0]) + w * RL_PAIRS * RL_LD;
    const int q = lane & 3, p = lane >> 2;
#pragma unroll
    for (int r = 0; r < RL_T * RL_E / RL_PAIRS; ++r) {
#pragma unroll
        for (int i = 0; i < RL_PAIRS; ++i) {
            const int pr = r * RL_PAIRS + i;
            rd[i * RL_LD + lane] = acc[pr / RL_E][pr % RL_E];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double v[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) v[m] = rd[p * RL_LD + q + 4 * m];
#pragma unroll
        for (int half = 8; half >= 1; half >>= 1)
#pragma unroll
            for (int m = 0; m < half; ++m) v[m] += v[m + half];
        double s = v[0];
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 1, 64);
        const int pr = r * RL_PAIRS + p;
        const int t = tb + wt * RL_T + pr / RL_E, e = eb + we * RL_E + pr % RL_E;
        if (q == 0 && t < T && e < E) {
            float f = (float)s;
            if (rb) f = f + rb[e];
            logits[(int64_t)t * E + e] = f;
        }
        __builtin_amdgcn_wave_barrier();   // the partials are read before the next round overwrites them
    }
}

// Expert selection for many tokens from logits[T, E]: one wave per token.
// CONV >= 0 (prefill): the wave also writes token t's f16 row of h for the
// gate_up GEMM (x_to_f16_row<CONV>), which saves that conversion its own
// launch.
struct F16Rows {
    const float *X;
    _Float16 *Xh;
    float *inv;
    int cols, ldh, vec;
    float *nrm2;   // each row's sum of squares (x_to_f16_row)
};
template <int CONV>
__global__ __launch_bounds__(256) void moe_topk_kernel(const float *__restrict__ logits, int T, int E, int k,
                                                       int32_t *__restrict__ topk_idx,
                                                       float *__restrict__ topk_w, F16Rows cv) {
    const int t = blockIdx.x * 4 + wave_id();
    if (t >= T) return;
    if constexpr (CONV >= 0)
        x_to_f16_row<CONV>(t, cv.X, cv.cols, cv.cols, nullptr, 1, T, cv.Xh, cv.ldh, cv.inv, cv.vec, 0, T, cv.nrm2);
    route_select_any(logits + (int64_t)t * E, E, k, t, topk_idx, topk_w, MoeTables{}, 0);
}

// Lanes of the wave whose (live) expert equals this lane's: one ballot per
// bit of the expert index (nbits = bits of E - 1), each lane keeping the
// lanes that agree with it on that bit.
__device__ __forceinline__ uint64_t match_lanes(int e, bool live, int nbits) {
    uint64_t m = __ballot(live);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t on = __ballot(bit);
        m &= bit ? on : ~on;
    }
    return m;
}

// Inclusive sum over the 64 lanes: DPP shifts inside each row of 16 lanes,
// then the totals of the rows below (read from lanes 15, 31, 47).
__device__ __forceinline__ int wave_incl_sum(int v, int lane) {
    const int r = lane & 15;
    int t;
    t = (int)dpp_u32<0x111>((uint32_t)v); if (r >= 1) v += t;
    t = (int)dpp_u32<0x112>((uint32_t)v); if (r >= 2) v += t;
    t = (int)dpp_u32<0x114>((uint32_t)v); if (r >= 4) v += t;
    t = (int)dpp_u32<0x118>((uint32_t)v); if (r >= 8) v += t;
    const int s0 = __builtin_amdgcn_readlane(v, 15), s1 = __builtin_amdgcn_readlane(v, 31);
    const int s2 = __builtin_amdgcn_readlane(v, 47);
    return v + (lane >= 16 ? s0 : 0) + (lane >= 32 ? s1 : 0) + (lane >= 48 ? s2 : 0);
}

constexpr int PERM_WAVES = 16;              // the permute's workgroup: 1024 threads
constexpr size_t PERM_LDS_MAX = 65536;

// LDS of the permute: cnt[16][E] and off[E + 1] ints, then (8-byte aligned)
// a region that holds first the wave-private lane masks [16][E] (u64, when
// `match`) and then the staged perm[N] (ints, when `stage`).
static inline size_t perm_lds_head(int64_t E) { return (size_t)((17 * E + 2) & ~1) * 4; }
static inline size_t perm_lds_bytes(int64_t E, int64_t N, bool match, bool stage) {
    const size_t a = match ? (size_t)(PERM_WAVES * E) * 8 : 0, b = stage ? (size_t)N * 4 : 0;
    return perm_lds_head(E) + (a > b ? a : b);
}

// Stable counting sort of the N assignments by expert in one workgroup of
// 1024 threads. Wave w owns the contiguous range [w per, (w+1) per):
//   1. per 64 assignments, the lanes with equal experts are matched -- MATCH:
//      every lane ORs its bit into the wave's LDS mask of its expert and reads
//      the mask back; else one ballot per expert-index bit. An assignment's
//      rank among its expert's assignments so far in the wave is kept (in
//      registers, or in pos[] as scratch until step 4 for long ranges) and the
//      wave's per-expert counts advance in LDS;
//   2. each expert's wave counts become exclusive bases in wave order (eight
//      lanes per expert, two waves each);
//   3. wave 0 scans the expert totals (lane l owns a contiguous run of
//      experts): offsets, counts, the active list and, for the expert GEMMs,
//      the tile list (tiles of tile_w consecutive perm positions per expert:
//      every expert's full tiles, then every expert's partial last tile);
//   4. every assignment lands at offset[e] + wave base + rank -- STAGE: in
//      LDS, copied out to perm[] in order afterwards (the scattered stores stay
//      off the one CU's address path).
// The result lists the assignments in (expert, a) order.
// sel_logits (not null; fewer than ROUTE_TILE_TOKENS tokens): the router
// wrote only the logits [N / k, E] (moe_route1_kernel); the waves first
// select each token's experts and gates (route_select, one wave per token)
// into idx / topk_w, then sort them.
template <bool MATCH, bool STAGE>
__global__ __launch_bounds__(1024) void moe_permute_kernel(int32_t *__restrict__ idx, int N, int E, MoeTables tb,
                                                           const float *__restrict__ sel_logits, int k,
                                                           float *__restrict__ topk_w) {
    extern __shared__ __align__(16) int ws[];
    constexpr int U = 8;                   // assignments per lane per batch of loads
    const int lane = lane_id(), w = wave_id();
    if (sel_logits) {
        for (int t = w; t < N / k; t += PERM_WAVES)
            route_select_any(sel_logits + (int64_t)t * E, E, k, t, idx, topk_w, tb, 0);
        __syncthreads();   // idx is read below by every wave
    }
    int *cnt = ws;
    int *off = ws + PERM_WAVES * E;
    const int head = (17 * E + 2) & ~1;
    uint64_t *masks = reinterpret_cast<uint64_t *>(ws + head);
    int *stage = ws + head;
    const int per = (N + PERM_WAVES - 1) / PERM_WAVES;
    const int a0 = min(N, w * per), a1 = min(N, a0 + per);
    // a wave range of at most 64 U assignments stays in registers (ev, rv)
    // until step 4; longer ranges keep the ranks in pos[]
    const bool held = a1 - a0 <= 64 * U;
    int ev[U], rv[U];
    // expert ids of the first batch, requested before the LDS is cleared
    // (every load is in bounds; lanes past a1 are masked where used)
#pragma unroll
    for (int u = 0; u < U; ++u) ev[u] = idx[min(a0 + 64 * u + lane, N - 1)];
    for (int i = threadIdx.x; i < PERM_WAVES * E; i += blockDim.x) cnt[i] = 0;
    if constexpr (MATCH)
        for (int i = threadIdx.x; i < PERM_WAVES * E; i += blockDim.x) masks[i] = 0ull;
    __syncthreads();
    const int nbits = E > 1 ? 32 - __builtin_clz((unsigned)(E - 1)) : 0;
    int *wc = cnt + w * E;
    uint64_t *wm = masks + w * E;
    for (int base = a0; base < a1; base += 64 * U) {
        if (base != a0) {
#pragma unroll
            for (int u = 0; u < U; ++u) ev[u] = idx[min(base + 64 * u + lane, N - 1)];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (base + 64 * u >= a1) break;   // uniform
            const int a = base + 64 * u + lane;
            const bool live = a < a1;
            const int e = ev[u];
            uint64_t m;
            if constexpr (MATCH) {
                if (live) __hip_atomic_fetch_or(wm + e, 1ull << lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
                m = live ? __hip_atomic_load(wm + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT) : 0ull;
            } else {
                m = match_lanes(e, live, nbits);
            }
            const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
            const int before = live ? wc[e] : 0;
            rv[u] = before + rank;
            if (live && !held) tb.pos[a] = rv[u];
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            // the highest matching lane advances the expert's count (and
            // clears its mask), after every lane has read both
            if (live && (m >> lane) == 1) {
                wc[e] = before + __builtin_popcountll(m);
                if constexpr (MATCH) wm[e] = 0ull;
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
    // step 2: lane j of the eight of expert e takes waves 2j and 2j + 1
    for (int eb = 0; eb < E; eb += 128) {
        const int e = eb + (int)(threadIdx.x >> 3), j = (int)(threadIdx.x & 7);
        const bool ok = e < E;
        const int c0 = ok ? cnt[2 * j * E + e] : 0, c1 = ok ? cnt[(2 * j + 1) * E + e] : 0;
        const int s = c0 + c1;
        int incl = s, t;
        t = (int)dpp_u32<0x111>((uint32_t)incl); if (j >= 1) incl += t;
        t = (int)dpp_u32<0x112>((uint32_t)incl); if (j >= 2) incl += t;
        t = (int)dpp_u32<0x114>((uint32_t)incl); if (j >= 4) incl += t;
        if (ok) {
            cnt[2 * j * E + e] = incl - s;           // exclusive within the expert, wave order
            cnt[(2 * j + 1) * E + e] = incl - s + c0;
            if (j == 7) off[e] = incl;               // the expert's total until the scan below
        }
    }
    __syncthreads();
    if (w == 0) {
        const int tw = tb.tile_w;
        const int pe = (E + 63) / 64;
        const int e0 = min(E, lane * pe), e1 = min(E, e0 + pe);
        int so = 0, sa = 0, sf = 0, sp = 0;
        for (int e = e0; e < e1; ++e) {
            const int c = off[e];
            so += c;
            sa += c > 0;
            if (tw > 0) {
                sf += c / tw;
                sp += c % tw != 0;
            }
        }
        // inclusive sums over the lanes, then exclusive starts of this lane's run;
        // the full tiles of every expert come first, the partial last tiles after
        // them: the expert GEMM grid starts the long tiles first and its last
        // workgroups are the short ones
        const int io = wave_incl_sum(so, lane), ia = wave_incl_sum(sa, lane);
        const int iff = tw > 0 ? wave_incl_sum(sf, lane) : 0, ip = tw > 0 ? wave_incl_sum(sp, lane) : 0;
        const int nfull = __builtin_amdgcn_readlane(iff, 63);
        int o = io - so, na = ia - sa, nf = iff - sf, np = nfull + ip - sp;
        for (int e = e0; e < e1; ++e) {
            const int c = off[e];
            off[e] = o;
            tb.offsets[e] = o;
            tb.counts[e] = c;
            if (c > 0) tb.active[na++] = e;
            if (tw > 0) {
                for (int p = 0; p + tw <= c; p += tw, ++nf) {
                    tb.tile_e[nf] = e;
                    tb.tile_p0[nf] = o + p;
                    tb.tile_n[nf] = tw;
                }
                if (c % tw) {
                    tb.tile_e[np] = e;
                    tb.tile_p0[np] = o + c - c % tw;
                    tb.tile_n[np] = c % tw;
                    ++np;
                }
            }
            o += c;
        }
        if (lane == 63) {
            off[E] = io;
            tb.offsets[E] = io;
            tb.n_active[0] = ia;
            if (tw > 0) tb.n_tiles[0] = iff + ip;
        }
    }
    __syncthreads();
    for (int base = a0; base < a1; base += 64 * U) {
        if (!held) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int a = min(base + 64 * u + lane, N - 1);
                ev[u] = idx[a];
                rv[u] = tb.pos[a];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int a = base + 64 * u + lane;
            if (a < a1) {
                const int p = off[ev[u]] + wc[ev[u]] + rv[u];
                if constexpr (STAGE)
                    stage[p] = a;
                else
                    tb.perm[p] = a;
                tb.pos[a] = p;
            }
        }
    }
    // the fused one-token kernel's counter block, whose error word
    // localai_hip_moe_error reads, is unused on the paths that permute
    for (int i = threadIdx.x; i < D1_WORDS; i += blockDim.x) tb.sync[i] = 0u;
    if constexpr (STAGE) {
        __syncthreads();
        for (int i = threadIdx.x; i < N; i += blockDim.x) tb.perm[i] = stage[i];
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

// gate_up: workgroup (i, slot) = gate tiles RT i .. RT i + RT - 1 (rows 16
// RT i ..) and the matching up tiles inter / 16 + RT i + t of the slot's
// expert; act[p, 16 (RT i + t) + n] = silu(g) * u (engine/zaya.py:303-306)
// for every perm position p of the expert. With zero != null the slot-0
// workgroups also clear zero[0 .. nzero) (the output that the down kernel
// then adds onto).
template <int TYPE, int SPW, int MAXT, int RT = 1>
__global__ __launch_bounds__(MAXT) void moe_mfma_gate_up(const uint8_t *__restrict__ Wt, int64_t mat_bytes, int nb,
                                                         int64_t inter, MoeTables tb, const float *__restrict__ h,
                                                         int64_t H, int k, float *__restrict__ zero,
                                                         int64_t nzero) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    if (zero && slot == 0) {
        const int64_t per = (nzero + gridDim.x - 1) / gridDim.x, c0 = blockIdx.x * per;
        for (int64_t c = c0 + threadIdx.x; c < c0 + per && c < nzero; c += blockDim.x) zero[c] = 0.0f;
    }
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x, tile_bytes = (int64_t)nb * mt_block_bytes(TYPE);
    const uint8_t *We = Wt + (int64_t)e * mat_bytes;
    const int64_t gtiles = inter / MT_ROWS;
    MtW<TYPE> w[2 * RT][SPW];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t gt = RT * i + t < gtiles ? RT * i + t : gtiles - 1;
        mt_load_tile<TYPE, SPW>(w[t], We + gt * tile_bytes, nb, sb0, nsb, lane);
        mt_load_tile<TYPE, SPW>(w[RT + t], We + (gtiles + gt) * tile_bytes, nb, sb0, nsb, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the expert's tokens; each next token's row is requested before the
    // current token's arithmetic
    const int n = tb.counts[e], base = tb.offsets[e];
    const int tok0 = tb.perm[base] / k;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], h + (int64_t)tok0 * H, nb, sb0, lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xn[1][SPW];
        if (j + 1 < n) mt_load_x<SPW>(xn[0], h + (int64_t)(tb.perm[p + 1] / k) * H, nb, sb0, lane);
        float *fin;
        mt_pass<TYPE, SPW, 2 * RT, 1>(w, xv, nsb, smem, fin);
        const int r = threadIdx.x;
        if (r < RT * MT_ROWS && RT * i * MT_ROWS + r < inter)
            tb.act[(int64_t)p * inter + RT * i * MT_ROWS + r] = silu(fin[r]) * fin[RT * MT_ROWS + r];
        if (j + 1 < n) {
#pragma unroll
            for (int kk = 0; kk < SPW; ++kk) xv[0][kk] = xn[0][kk];
        }
    }
}

// down: workgroup (i, slot) = hidden tiles RT i .. RT i + RT - 1 of the
// slot's expert; ysl[p, r] for those rows r and every perm position p of the
// expert, or with out != null (k <= 2, out cleared by gate_up) out[t, r] +=
// gate * y for the
// token t of position p: two additions onto zero give the same sum in either
// order, so the combine is folded in without changing the result's bits
template <int TYPE, int SPW, int MAXT, int RT = 1>
__global__ __launch_bounds__(MAXT) void moe_mfma_down(const uint8_t *__restrict__ Wt, int64_t mat_bytes, int nb,
                                                      int64_t hidden, MoeTables tb, int64_t inter,
                                                      float *__restrict__ out, const float *__restrict__ topk_w,
                                                      int k) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int n = tb.counts[e], base = tb.offsets[e];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], tb.act + (int64_t)base * inter, nb, sb0, lane);
    const int64_t tiles = (hidden + MT_ROWS - 1) / MT_ROWS;
    MtW<TYPE> w[RT][SPW];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t ti = RT * i + t < tiles ? RT * i + t : tiles - 1;
        mt_load_tile<TYPE, SPW>(w[t], Wt + (int64_t)e * mat_bytes + ti * nb * mt_block_bytes(TYPE), nb, sb0, nsb,
                                lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xn[1][SPW];
        if (j + 1 < n) mt_load_x<SPW>(xn[0], tb.act + (int64_t)(p + 1) * inter, nb, sb0, lane);
        float *fin;
        mt_pass<TYPE, SPW, RT, 1>(w, xv, nsb, smem, fin);
        const int r = threadIdx.x;
        const int64_t row = RT * i * MT_ROWS + r;
        if (r < RT * MT_ROWS && row < hidden) {
            if (out) {
                const int a = tb.perm[p];
                atomicAdd(out + (int64_t)(a / k) * hidden + row, topk_w[a] * fin[r]);
            } else {
                tb.ysl[(int64_t)p * hidden + row] = fin[r];
            }
        }
        if (j + 1 < n) {
#pragma unroll
            for (int kk = 0; kk < SPW; ++kk) xv[0][kk] = xn[0][kk];
        }
    }
}

// Rows of more than 32 blocks of 256 (up to 64): each wave's eight blocks
// stream through two register sets (mt_pass_pipe) for every token instead
// of being held, x is read for each token after the previous pass, and
// gate_up runs its gate and up tiles as two passes; otherwise as
// moe_mfma_gate_up / moe_mfma_down with one row tile per workgroup.
template <int TYPE, int SPW>
__global__ __launch_bounds__(512) void moe_mfma_gate_up_pipe(const uint8_t *__restrict__ Wt, int64_t mat_bytes,
                                                              int nb, int64_t inter, MoeTables tb,
                                                              const float *__restrict__ h, int64_t H, int k,
                                                              float *__restrict__ zero, int64_t nzero) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    if (zero && slot == 0) {
        const int64_t per = (nzero + gridDim.x - 1) / gridDim.x, c0 = blockIdx.x * per;
        for (int64_t c = c0 + threadIdx.x; c < c0 + per && c < nzero; c += blockDim.x) zero[c] = 0.0f;
    }
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x, tile_bytes = (int64_t)nb * mt_block_bytes(TYPE);
    const uint8_t *We = Wt + (int64_t)e * mat_bytes;
    const int64_t gtiles = inter / MT_ROWS;
    const uint8_t *const tg[1] = {We + i * tile_bytes}, *const tu[1] = {We + (gtiles + i) * tile_bytes};
    const int n = tb.counts[e], base = tb.offsets[e];
    const int r = threadIdx.x;
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xv[SPW];
        mt_load_x<SPW>(xv, h + (int64_t)(tb.perm[p] / k) * H, nb, sb0, lane);
        float *fin;
        mt_pass_pipe<TYPE, SPW, 1>(tg, nb, sb0, nsb, xv, smem, fin);
        const float gv = r < MT_ROWS ? fin[r] : 0.0f;
        mt_pass_pipe<TYPE, SPW, 1>(tu, nb, sb0, nsb, xv, smem, fin);
        if (r < MT_ROWS) tb.act[(int64_t)p * inter + i * MT_ROWS + r] = silu(gv) * fin[r];
    }
}

template <int TYPE, int SPW>
__global__ __launch_bounds__(512) void moe_mfma_down_pipe(const uint8_t *__restrict__ Wt, int64_t mat_bytes, int nb,
                                                           int64_t hidden, MoeTables tb, int64_t inter,
                                                           float *__restrict__ out, const float *__restrict__ topk_w,
                                                           int k) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int slot = blockIdx.y;
    if (slot >= tb.n_active[0]) return;
    const int e = tb.active[slot];
    const int n = tb.counts[e], base = tb.offsets[e];
    const int lane = lane_id(), sb0 = wave_id() * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t i = blockIdx.x;
    const uint8_t *const tl[1] = {Wt + (int64_t)e * mat_bytes + i * nb * mt_block_bytes(TYPE)};
    const int r = threadIdx.x;
    const int64_t row = i * MT_ROWS + r;
    for (int j = 0; j < n; ++j) {
        const int p = base + j;
        float4 xv[SPW];
        mt_load_x<SPW>(xv, tb.act + (int64_t)p * inter, nb, sb0, lane);
        float *fin;
        mt_pass_pipe<TYPE, SPW, 1>(tl, nb, sb0, nsb, xv, smem, fin);
        if (r < MT_ROWS && row < hidden) {
            if (out) {
                const int a = tb.perm[p];
                atomicAdd(out + (int64_t)(a / k) * hidden + row, topk_w[a] * fin[r]);
            } else {
                tb.ysl[(int64_t)p * hidden + row] = fin[r];
            }
        }
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

// The same sums for K = k known at compile time and H % 4 == 0 (16-byte
// rows): every one of the token's K rows is requested before the first is
// added (the loop above waits for each load in turn), four columns per
// thread; the additions keep the top-k order, so the bits are the same.
template <int K>
__global__ void moe_combine_vec_kernel(const float *__restrict__ ysl, const int32_t *__restrict__ pos,
                                       const float *__restrict__ topk_w, int H, float *__restrict__ out) {
    const int t = blockIdx.y;
    const int c4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * c4 >= H) return;
    typedef float f4v __attribute__((ext_vector_type(4)));
    f4v y[K];   // expert output rows, each read once
#pragma unroll
    for (int j = 0; j < K; ++j)
        y[j] = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(ysl + (int64_t)pos[t * K + j] * H) + c4);
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const float w = topk_w[t * K + j];
        s = make_float4(__builtin_fmaf(w, y[j].x, s.x), __builtin_fmaf(w, y[j].y, s.y), __builtin_fmaf(w, y[j].z, s.z),
                        __builtin_fmaf(w, y[j].w, s.w));
    }
    reinterpret_cast<float4 *>(out + (int64_t)t * H)[c4] = s;
}

// ------------------------------------------------- one-token decode, fused

// The expert part of the MoE layer for one token with k <= 2 in one launch,
// after topk_idx / topk_w were written (by the permutation's selection, or by
// the caller: localai_hip_moe_experts1) and the counter block zeroed.
// Workgroup r:
//   r < n_gu          gate_up tile i of slot s (n_gu = k * inter / 16): the
//                     expert's weights, act[s] rows; clears its share of out;
//                     counts itself done
//   r >= n_gu         down tile i of slot s: weights requested at once (they
//                     stream beside gate_up's), then waits for every gate_up
//                     tile; out += gate * y
// Workgroups start in id order, so every gate_up tile has started before a
// down tile waits (and every wait is bounded). Two additions onto zero give
// the same sum in either order, so out does not depend on which down tile
// lands first. 8 waves; SPWG / SPWD super-blocks per wave for gate_up / down.
// LDS: the mt_pass regions.
// sel_logits (not null; E <= 64): the router wrote only the logits
// (moe_route1_kernel) and each workgroup selects the experts itself, before
// anything else; topk_idx / topk_w then receive the selection, and the
// routing tables (counts, offsets, active, perm, pos) come from the first
// down tile.
// SKIP: skip is the route index that stands for "no expert" (ZAYA's skip
// route, engine/zaya.py:297-301): its slot adds gate * h instead of an
// expert output; its gate_up tiles read no weights but still clear and
// count. A template flag because the test costs the plain top-k layer
// 0.5 us (13.2 vs 12.7 us, Q6_K, hidden 2048, top-2).
// Failures are loud: an expert index outside [0, E) that is not the skip
// route, or a wait that runs out (spin polls), sets a bit of the error word
// (sync + D1_ERROR) and makes the affected rows of out NaN. count = 0 keeps
// the gate_up tiles from counting themselves done (a test of the error path:
// every wait then runs out and every workgroup still exits).
template <int TYPE, int SPWG, int SPWD, bool SKIP>
__global__ __launch_bounds__(512) void moe_decode1_kernel(
    const float *__restrict__ h, int H, int E, int k, const uint8_t *__restrict__ gu_t, int64_t gu_bytes, int nbg,
    int64_t inter, const uint8_t *__restrict__ dn_t, int64_t dn_bytes, int nbd, const int32_t *topk_idx,
    const float *topk_w, float *__restrict__ out, MoeTables tb, uint32_t *__restrict__ sync, int skip, int spin,
    int count, const float *__restrict__ sel_logits) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int flag;
    __shared__ int sel_idx[2];
    __shared__ float sel_w[2];
    const int r = blockIdx.x;
    const int lane = lane_id(), w = wave_id();
    const int gtiles = (int)(inter / MT_ROWS), dtiles = (H + MT_ROWS - 1) / MT_ROWS;
    const int n_gu = k * gtiles;
    if (sel_logits) {
        // the experts come from the E logits of moe_route1_kernel: every
        // workgroup selects them itself (route_select, the router's own
        // rule); workgroup 0 also writes them out
        if (w == 0) {
            // the first down tile (which waits anyway) also writes the routing tables
            route_select<1>(sel_logits, E, k, 0, sel_idx, sel_w, tb, r == n_gu);
            if (r == 0 && lane < k) {
                const_cast<int32_t *>(topk_idx)[lane] = sel_idx[lane];
                const_cast<float *>(topk_w)[lane] = sel_w[lane];
            }
        }
        __syncthreads();
        topk_idx = sel_idx;
        topk_w = sel_w;
    }
    if (r < n_gu) {
        const int s = r / gtiles, i = r % gtiles;
        const int n = threadIdx.x;
        const int idx = topk_idx[s];   // the same for the whole workgroup
        const bool is_skip = SKIP && idx == skip;
        if (!is_skip && (idx < 0 || idx >= E)) {
            if (n == 0 && i == 0) d1_error(sync, D1_ERR_INDEX);
        } else if (!is_skip) {
            const int sb0 = w * SPWG, nsb = mt_nsb(nbg, sb0, SPWG);
            const int e = idx;
            const uint8_t *We = gu_t + (int64_t)e * gu_bytes;
            const int64_t tb_bytes = (int64_t)nbg * mt_block_bytes(TYPE);
            MtW<TYPE> wt[2][SPWG];
            mt_load_tile<TYPE, SPWG>(wt[0], We + i * tb_bytes, nbg, sb0, nsb, lane);
            mt_load_tile<TYPE, SPWG>(wt[1], We + (gtiles + i) * tb_bytes, nbg, sb0, nsb, lane);
            float4 xv[1][SPWG];
            mt_load_x<SPWG>(xv[0], h, nbg, sb0, lane);
            float *fin;
            mt_pass<TYPE, SPWG, 2, 1>(wt, xv, nsb, smem, fin);
            if (n < MT_ROWS) d1_put(tb.act + (int64_t)s * inter + i * MT_ROWS + n, silu(fin[n]) * fin[MT_ROWS + n]);
        }
        const int per = (H + n_gu - 1) / n_gu;   // this tile's share of out
        for (int c = r * per + n; c < (r + 1) * per && c < H; c += blockDim.x) d1_put(out + c, 0.0f);
        d1_drain();
        __syncthreads();
        if (threadIdx.x == 0 && count) d1_count(sync, r, n_gu);
        return;
    }
    const int j = r - n_gu, s = j / dtiles, i = j % dtiles;
    const float gate = topk_w[s];
    const int idx = topk_idx[s];
    const float nan = __builtin_nanf("");
    if (SKIP && idx == skip) {   // out += gate * h on this tile's rows
        const bool ok = d1_wait_done(sync, &flag, spin);
        const int row = i * MT_ROWS + (int)threadIdx.x;
        if (threadIdx.x < MT_ROWS && row < H) atomicAdd(out + row, ok ? gate * h[row] : nan);
        return;
    }
    const bool bad = idx < 0 || idx >= E;   // flagged by the slot's gate_up tiles
    const int sb0 = w * SPWD, nsb = mt_nsb(nbd, sb0, SPWD);
    const int e = bad ? 0 : idx;
    MtW<TYPE> wt[1][SPWD];
    mt_load_tile<TYPE, SPWD>(wt[0], dn_t + (int64_t)e * dn_bytes + i * (int64_t)nbd * mt_block_bytes(TYPE), nbd, sb0,
                             nsb, lane);
    const bool ok = d1_wait_done(sync, &flag, spin) && !bad;
    float4 xv[1][SPWD];
    d1_load_x<SPWD>(xv[0], tb.act + (int64_t)s * inter, nbd, sb0, lane);
    float *fin;
    mt_pass<TYPE, SPWD, 1, 1>(wt, xv, nsb, smem, fin);
    const int n = threadIdx.x;
    if (n < MT_ROWS && i * MT_ROWS + n < H) atomicAdd(out + i * MT_ROWS + n, ok ? gate * fin[n] : nan);
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

// Whether the prefill gate_up GEMM writes the down GEMM's f16 rows itself
// (on the tile form, with the handle's row norms, rows without padding);
// else it writes fp32 SiLU * up rows and x_to_f16 converts them.
static bool moe_gate_up_f16_out(const localai_qmat *gu, int64_t I) {
    return gu->tiles && gu->row_norm && I % MT_ROWS == 0 && f16_stride(I) == I;
}

// Byte offsets of the workspace's tables, each 256-byte aligned (the expert
// GEMM tables only from MOE_GEMM_TOKENS tokens on; -1 otherwise).
MoeLayout moe_layout(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const int64_t N = T * k;
    MoeLayout L;
    int64_t p = 0;
    auto take = [&](int64_t n) { const int64_t q = p; p += (int64_t)align256((size_t)n); return q; };
    L.logits = take(T * E * 4);
    L.sync = take(D1_WORDS * 4);
    L.counts = take(E * 4);
    L.offsets = take((E + 1) * 4);
    L.active = take(E * 4);
    L.n_active = take(4);
    L.perm = take(N * 4);
    L.pos = take(N * 4);
    L.act = take(N * I * 4);
    L.ysl = take(N * H * 4);
    L.max_tiles = 0;
    L.tile_e = L.tile_p0 = L.tile_n = L.n_tiles = L.xh_gu = L.inv_gu = L.hn2 = L.xh_dn = L.inv_dn = -1;
    if (T >= MOE_GEMM_TOKENS) {
        L.max_tiles = moe_max_tiles(N, E, moe_gemm_tile());
        L.tile_e = take(L.max_tiles * 4);
        L.tile_p0 = take(L.max_tiles * 4);
        L.tile_n = take(L.max_tiles * 4);
        L.n_tiles = take(4);
        L.xh_gu = take(T * f16_stride(H) * 2);
        L.inv_gu = take(T * 4);
        L.hn2 = take(T * 4);
        L.xh_dn = take(N * f16_stride(I) * 2);
        L.inv_dn = take(N * 4);
    }
    L.bytes = p;
    return L;
}

size_t moe_workspace_bytes(int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    return (size_t)moe_layout(T, E, k, H, I).bytes;
}

static MoeTables carve(void *ws, int64_t T, int64_t E, int64_t k, int64_t H, int64_t I) {
    const MoeLayout L = moe_layout(T, E, k, H, I);
    uint8_t *p = (uint8_t *)ws;
    MoeTables tb{};
    tb.logits = (float *)(p + L.logits);
    tb.sync = (uint32_t *)(p + L.sync);
    tb.counts = (int32_t *)(p + L.counts);
    tb.offsets = (int32_t *)(p + L.offsets);
    tb.active = (int32_t *)(p + L.active);
    tb.n_active = (int32_t *)(p + L.n_active);
    tb.perm = (int32_t *)(p + L.perm);
    tb.pos = (int32_t *)(p + L.pos);
    tb.act = (float *)(p + L.act);
    tb.ysl = (float *)(p + L.ysl);
    tb.tile_w = 0;
    if (L.max_tiles > 0) {
        tb.tile_w = moe_gemm_tile();
        tb.max_tiles = (int)L.max_tiles;
        tb.tile_e = (int32_t *)(p + L.tile_e);
        tb.tile_p0 = (int32_t *)(p + L.tile_p0);
        tb.tile_n = (int32_t *)(p + L.tile_n);
        tb.n_tiles = (int32_t *)(p + L.n_tiles);
        tb.xh_gu = (_Float16 *)(p + L.xh_gu);
        tb.inv_gu = (float *)(p + L.inv_gu);
        tb.hn2 = (float *)(p + L.hn2);
        tb.xh_dn = (_Float16 *)(p + L.xh_dn);
        tb.inv_dn = (float *)(p + L.inv_dn);
    }
    return tb;
}

template <int T, bool GATE_UP, int NT>
static void launch_grouped_t(const localai_qmat *m, const uint8_t *planes, int lpr, int waves, const MoeTables &tb,
                             const float *xsrc, int64_t x_stride, int k, int slots, int64_t max_tokens,
                             hipStream_t s) {
    const lq_geom &g = m->g;
    const int64_t half = GATE_UP ? g.rows / 2 : g.rows;
    const int64_t tile = (int64_t)(moe_rows<T, NT>() / (GATE_UP ? 2 : 1)) * (64 / lpr);
    dim3 grid((unsigned)((half + tile - 1) / tile), slots, (unsigned)((max_tokens + NT - 1) / NT)),
        block(64 * waves);
    const size_t lds = (size_t)waves * NT * 16 * lpr * 16;
    if (lpr == 16)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 16, NT>), grid, block, lds, s, planes, g, tb, xsrc,
                           x_stride, k);
    else if (lpr == 32)
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 32, NT>), grid, block, lds, s, planes, g, tb, xsrc,
                           x_stride, k);
    else
        hipLaunchKernelGGL((moe_grouped_kernel<T, GATE_UP, 64, NT>), grid, block, lds, s, planes, g, tb, xsrc,
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
    int st;
    const uint8_t *planes = qmat_planes(m, s, &st);   // this path reads the row planes
    if (!planes) return st;
    switch (g.type) {
#define LQ_G(TT)                                                                                      \
    case TT:                                                                                          \
        if (nt == 2) launch_grouped_t<TT, GATE_UP, 2>(m, planes, lpr, waves, tb, xsrc, x_stride, k, slots, max_tokens, s); \
        else launch_grouped_t<TT, GATE_UP, 1>(m, planes, lpr, waves, tb, xsrc, x_stride, k, slots, max_tokens, s);        \
        break;
        LQ_G(LQ_Q4_K) LQ_G(LQ_Q5_K) LQ_G(LQ_Q6_K) LQ_G(LQ_Q8_0) LQ_G(LQ_Q4_0)
#undef LQ_G
        default: return fail(LOCALAI_ETYPE, "moe: unsupported expert type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// MFMA decode path: both expert tensors in the tile form (Q4_K, Q6_K, or
// Q8_0 with rows of whole 256-value blocks, since the kernels read x 256
// values a block) with K <= 64 blocks of 256: one block per wave (up to 16
// waves) for K <= 16, four per wave for K <= 32 (up to 8 waves, room for
// the registers), eight per wave streamed through two register sets for
// K <= 64 (8 waves; moe_mfma_gate_up_pipe / moe_mfma_down_pipe).
static bool moe_mfma_ok(const localai_qmat *gu, const localai_qmat *dn, const float *h, int64_t H, int64_t I) {
    const bool q80 = gu->g.type == LQ_Q8_0;
    // the streamed kernels' LDS (8 waves of eight staged blocks, ~76 KB)
    const bool lds = (mt_nsb(gu->g) <= 32 && mt_nsb(dn->g) <= 32) ||
                     mt_lds_bytes(gu->g.type, 8, 8, 1, 1) <= max_lds_per_block();
    return gu->tiles && dn->tiles && gu->g.type == dn->g.type && mt_nsb(gu->g) <= 64 && mt_nsb(dn->g) <= 64 && lds &&
           (!q80 || (H % 256 == 0 && I % 256 == 0)) && (reinterpret_cast<uintptr_t>(h) & 15) == 0 &&
           I % MT_ROWS == 0 && gu->g.cols == H && dn->g.cols == I;
}

// The fused one-token kernel: at most 32 blocks of 256 per row (four per
// wave of its 8 waves)
static bool moe_decode1_ok(const localai_qmat *gu, const localai_qmat *dn) {
    return mt_nsb(gu->g) <= 32 && mt_nsb(dn->g) <= 32;
}

// Whether launch_moe would have to build the row planes of gu or dn (a
// hipMalloc, qmat_planes) for these sizes: the same path choice as
// launch_moe (expert GEMMs from MOE_GEMM_TOKENS tokens on, read the tile
// form where there is one; below that the MFMA decode kernels, else the
// grouped VALU kernels over the row planes), true only where the handle does
// not hold the planes yet.
bool moe_would_build_planes(const float *h, int64_t T, int64_t H, const localai_qmat *gu, const localai_qmat *dn) {
    const int64_t I = gu->g.rows / 2;
    bool need_gu, need_dn;
    if (T >= MOE_GEMM_TOKENS) {
        need_gu = !(gu->tiles && I % MT_ROWS == 0);
        need_dn = !dn->tiles;
    } else {
        need_gu = need_dn = !moe_mfma_ok(gu, dn, h, H, I);
    }
    auto missing = [](const localai_qmat *m) { return __atomic_load_n(&m->data, __ATOMIC_ACQUIRE) == nullptr; };
    return (need_gu && missing(gu)) || (need_dn && missing(dn));
}

// Grouped decode kernels. gate_up: one super-block per wave (up to 16
// waves), or four past 16 super-blocks, one gate and one up tile per
// workgroup. down: at most 8 waves of SPW super-blocks and RT = 2 row tiles
// per workgroup (~100 KB of weights each): ZAYA down at 8 tokens 24.8 ->
// 20.6 us against 16 one-super-block waves on one tile; the same shape for
// gate_up (2 gate + 2 up tiles, 154 VGPRs) was slower, 33.0 -> 34.3 us.
template <int TYPE, int SPW, int MAXT, int RT>
static void launch_moe_mfma_st(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                               int64_t H, int64_t I, int k, int slots, float *out, const float *topk_w, int64_t T,
                               bool gate_up, hipStream_t s) {
    if (gate_up) {
        const int nb = (int)mt_nsb(gu->g), waves = (nb + SPW - 1) / SPW;
        const int64_t groups = (I / MT_ROWS + RT - 1) / RT;
        hipLaunchKernelGGL((moe_mfma_gate_up<TYPE, SPW, MAXT, RT>), dim3((unsigned)groups, slots), dim3(64 * waves),
                           mt_lds_bytes(TYPE, waves, SPW, 1, 2 * RT), s, gu->tiles, gu->tile_bytes, nb, I, tb, h, H, k,
                           out, T * H);
    } else {
        const int nb = (int)mt_nsb(dn->g), waves = (nb + SPW - 1) / SPW;
        const int64_t groups = ((H + MT_ROWS - 1) / MT_ROWS + RT - 1) / RT;
        hipLaunchKernelGGL((moe_mfma_down<TYPE, SPW, MAXT, RT>), dim3((unsigned)groups, slots), dim3(64 * waves),
                           mt_lds_bytes(TYPE, waves, SPW, 1, RT), s, dn->tiles, dn->tile_bytes, nb, H, tb, I, out,
                           topk_w, k);
    }
}

// rows of 33 .. 64 blocks: moe_mfma_gate_up_pipe / moe_mfma_down_pipe, 8 waves
// of eight blocks
template <int TYPE>
static void launch_moe_mfma_pipe(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                                 int64_t H, int64_t I, int k, int slots, float *out, const float *topk_w, int64_t T,
                                 bool gate_up, hipStream_t s) {
    if (gate_up) {
        const int nb = (int)mt_nsb(gu->g), waves = (nb + 7) / 8;
        hipLaunchKernelGGL((moe_mfma_gate_up_pipe<TYPE, 8>), dim3((unsigned)(I / MT_ROWS), slots), dim3(64 * waves),
                           mt_lds_bytes(TYPE, waves, 8, 1, 1), s, gu->tiles, gu->tile_bytes, nb, I, tb, h, H, k, out,
                           T * H);
    } else {
        const int nb = (int)mt_nsb(dn->g), waves = (nb + 7) / 8;
        hipLaunchKernelGGL((moe_mfma_down_pipe<TYPE, 8>), dim3((unsigned)((H + MT_ROWS - 1) / MT_ROWS), slots),
                           dim3(64 * waves), mt_lds_bytes(TYPE, waves, 8, 1, 1), s, dn->tiles, dn->tile_bytes, nb, H,
                           tb, I, out, topk_w, k);
    }
}

template <int TYPE>
static int launch_moe_mfma_t(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                             int64_t H, int64_t I, int k, int slots, float *out, const float *topk_w, int64_t T,
                             hipStream_t s) {
    // at most 64 blocks of 256 per row for both (moe_mfma_ok)
    const int64_t ng = mt_nsb(gu->g), nd = mt_nsb(dn->g);
    if (ng <= 16)
        launch_moe_mfma_st<TYPE, 1, 1024, 1>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, true, s);
    else if (ng <= 32)
        launch_moe_mfma_st<TYPE, 4, 512, 1>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, true, s);
    else
        launch_moe_mfma_pipe<TYPE>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, true, s);
    LQ_HIP(hipGetLastError());
    if (nd <= 8)
        launch_moe_mfma_st<TYPE, 1, 512, 2>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, false, s);
    else if (nd <= 16)
        launch_moe_mfma_st<TYPE, 2, 512, 2>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, false, s);
    else if (nd <= 32)
        launch_moe_mfma_st<TYPE, 4, 512, 1>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, false, s);
    else
        launch_moe_mfma_pipe<TYPE>(gu, dn, tb, h, H, I, k, slots, out, topk_w, T, false, s);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// super-blocks per wave of an 8-wave workgroup over nb blocks (nb <= 32)
static int d1_spw(int64_t nb) {
    const int64_t v = (nb + 7) / 8;
    return v <= 1 ? 1 : v <= 2 ? 2 : 4;
}

// Test controls of the fused kernel's waits (localai_hip_debug_fused_wait):
// the polling bound, and whether the gate_up tiles count themselves done.
static std::atomic<int> g_d1_spin{D1_SPIN_LIMIT}, g_d1_count{1};

int set_fused_wait(int spin, int count) {
    g_d1_spin.store(spin > 0 ? spin : D1_SPIN_LIMIT);
    g_d1_count.store(count ? 1 : 0);
    return LOCALAI_OK;
}

int moe_error_word(const void *ws, int64_t T, int64_t E, hipStream_t s, uint32_t *word) {
    const uint32_t *sync = (const uint32_t *)((const uint8_t *)ws + moe_layout(T, E, 1, 1, 1).sync);
    LQ_HIP(hipStreamSynchronize(s));
    LQ_HIP(hipMemcpy(word, sync + D1_ERROR, 4, hipMemcpyDeviceToHost));
    return LOCALAI_OK;
}

template <int TYPE, int SG, int SD>
static void launch_decode1_k(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                             int64_t H, int64_t E, int k, int64_t I, const int32_t *topk_idx, const float *topk_w,
                             float *out, int skip, hipStream_t s, const float *sel_logits) {
    const size_t a = mt_lds_bytes(TYPE, 8, SG, 1, 2), b = mt_lds_bytes(TYPE, 8, SD, 1, 1);
    const unsigned grid = (unsigned)(k * (I / MT_ROWS) + k * ((H + MT_ROWS - 1) / MT_ROWS));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(grid), dim3(512), a > b ? a : b, s, h, (int)H, (int)E, k, gu->tiles,
                           gu->tile_bytes, (int)mt_nsb(gu->g), I, dn->tiles, dn->tile_bytes, (int)mt_nsb(dn->g), topk_idx,
                           topk_w, out, tb, tb.sync, skip, g_d1_spin.load(), g_d1_count.load(), sel_logits);
    };
    if (skip >= 0)
        go(moe_decode1_kernel<TYPE, SG, SD, true>);
    else
        go(moe_decode1_kernel<TYPE, SG, SD, false>);
}

template <int TYPE>
static int launch_decode1_t(const localai_qmat *gu, const localai_qmat *dn, const MoeTables &tb, const float *h,
                            int64_t H, int64_t E, int k, int64_t I, const int32_t *topk_idx, const float *topk_w,
                            float *out, hipStream_t s, int skip = -1, const float *sel_logits = nullptr) {
    const int sg = d1_spw(mt_nsb(gu->g)), sd = d1_spw(mt_nsb(dn->g));
#define LQ_D1(SG, SD)                                                                                       \
    if (sg == SG && sd == SD)                                                                               \
        launch_decode1_k<TYPE, SG, SD>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, skip, s, sel_logits);
    LQ_D1(1, 1) else LQ_D1(1, 2) else LQ_D1(1, 4) else LQ_D1(2, 1) else LQ_D1(2, 2) else LQ_D1(2, 4)
    else LQ_D1(4, 1) else LQ_D1(4, 2) else LQ_D1(4, 4)
#undef LQ_D1
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_moe(const float *h, int64_t T, int64_t H, const float *rw, const float *rb, int64_t E, int k,
               const localai_qmat *gu, const localai_qmat *dn, float *out, int32_t *topk_idx, float *topk_w,
               void *ws, hipStream_t s) {
    const int64_t I = gu->g.rows / 2;
    MoeTables tb = carve(ws, T, E, k, H, I);
    const bool one = T == 1 && tb.tile_w == 0;
    // the fused expert kernel clears out while other workgroups still read h
    const bool apart = out + T * H <= h || h + T * H <= out;
    if (one && k <= 2 && E <= 64 && apart && moe_mfma_ok(gu, dn, h, H, I) && moe_decode1_ok(gu, dn)) {
        // one token through the fused expert kernel: the router writes only
        // the logits and the expert kernel selects
        if (H % (256 * ROUTE_CH))
            hipLaunchKernelGGL(moe_route1_kernel<true>, dim3((unsigned)E), dim3(64), 0, s, h, (int)H, rw, rb,
                               tb.logits, tb.sync);
        else
            hipLaunchKernelGGL(moe_route1_kernel<false>, dim3((unsigned)E), dim3(64), 0, s, h, (int)H, rw, rb,
                               tb.logits, tb.sync);
        LQ_HIP(hipGetLastError());
        switch (gu->g.type) {
            case LQ_Q6_K:
                return launch_decode1_t<LQ_Q6_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, -1, tb.logits);
            case LQ_Q8_0:
                return launch_decode1_t<LQ_Q8_0>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, -1, tb.logits);
            default:
                return launch_decode1_t<LQ_Q4_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, -1, tb.logits);
        }
    }
    bool h_f16_done = false;   // the f16 rows of h for the expert GEMMs written
    if (T >= ROUTE_TILE_TOKENS) {
        const bool part = H % 256 != 0;
        const dim3 lgrid((unsigned)((T + RL_TOK - 1) / RL_TOK), (unsigned)((E + RL_EXP - 1) / RL_EXP));
        if (part)
            hipLaunchKernelGGL(moe_route_logits_kernel<true>, lgrid, dim3(64 * RL_NW), 0, s, h, (int)T, (int)H, rw, rb,
                               (int)E, tb.logits);
        else
            hipLaunchKernelGGL(moe_route_logits_kernel<false>, lgrid, dim3(64 * RL_NW), 0, s, h, (int)T, (int)H, rw, rb,
                               (int)E, tb.logits);
        LQ_HIP(hipGetLastError());
        const dim3 tgrid((unsigned)((T + 3) / 4));
        if (tb.tile_w > 0 && gu->g.cols == H && H % 8 == 0 && f16_stride(H) <= 8 * 64 * 8) {
            // prefill: the f16 rows of h that gate_up reads come with the selection
            const F16Rows cv{h,   tb.xh_gu, tb.inv_gu, (int)H, (int)f16_stride(H), (int)((uintptr_t)h % 16 == 0 && H % 4 == 0),
                             tb.hn2};
            const int per = (int)((f16_stride(H) / 8 + 63) / 64);
            auto go = [&](auto kern) {
                hipLaunchKernelGGL(kern, tgrid, dim3(256), 0, s, tb.logits, (int)T, (int)E, k, topk_idx, topk_w, cv);
            };
            if (per <= 1) go(moe_topk_kernel<1>);
            else if (per <= 2) go(moe_topk_kernel<2>);
            else if (per <= 4) go(moe_topk_kernel<4>);
            else go(moe_topk_kernel<8>);
            h_f16_done = true;
        } else {
            hipLaunchKernelGGL(moe_topk_kernel<-1>, tgrid, dim3(256), 0, s, tb.logits, (int)T, (int)E, k, topk_idx,
                               topk_w, F16Rows{});
        }
    } else {
        // few tokens: the logits over (expert, token) one-wave workgroups; the
        // permutation selects the experts
        const dim3 rgrid((unsigned)E, (unsigned)T);
        if (H % (256 * ROUTE_CH))
            hipLaunchKernelGGL(moe_route1_kernel<true>, rgrid, dim3(64), 0, s, h, (int)H, rw, rb, tb.logits, tb.sync);
        else
            hipLaunchKernelGGL(moe_route1_kernel<false>, rgrid, dim3(64), 0, s, h, (int)H, rw, rb, tb.logits, tb.sync);
    }
    LQ_HIP(hipGetLastError());
    {
        const int64_t N = T * k;
        const bool match = perm_lds_bytes(E, N, true, false) <= PERM_LDS_MAX;
        const bool stage = perm_lds_bytes(E, N, match, true) <= PERM_LDS_MAX;
        const size_t sh2 = perm_lds_bytes(E, N, match, stage);
        const float *sel = T < ROUTE_TILE_TOKENS ? tb.logits : nullptr;
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(1), dim3(1024), sh2, s, topk_idx, (int)N, (int)E, tb, sel, k, topk_w);
        };
        if (match)
            stage ? go(moe_permute_kernel<true, true>) : go(moe_permute_kernel<true, false>);
        else
            stage ? go(moe_permute_kernel<false, true>) : go(moe_permute_kernel<false, false>);
        LQ_HIP(hipGetLastError());
    }
    const int slots = (int)(E < T * k ? E : T * k);
    if (tb.tile_w > 0) {
        // prefill: gathered f16 token rows -> expert GEMMs on MFMA
        const int64_t N = T * k;
        if (gu->g.cols != H || dn->g.cols != I) return fail(LOCALAI_EARG, "moe: expert shapes");
        // gate_up reads the f16 rows of h through the permutation (perm[p] / k)
        if (!h_f16_done)
            if (int st = launch_x_to_f16(h, H, H, nullptr, 1, T, tb.xh_gu, f16_stride(H), tb.inv_gu, s, 0, tb.hn2))
                return st;
        // the expert GEMMs read the tile form where there is one (gate_up
        // with inter a multiple of 16), else the row planes
        int st = LOCALAI_OK;
        const bool gu_tiled = gu->tiles && I % MT_ROWS == 0;
        const uint8_t *wgu = gu_tiled ? nullptr : qmat_planes(gu, s, &st);
        if (st) return st;
        const uint8_t *wdn = dn->tiles ? nullptr : qmat_planes(dn, s, &st);
        if (st) return st;
        // on the tile form, gate_up writes the down GEMM's f16 rows itself
        const MoeF16Out direct{tb.xh_dn, f16_stride(I), tb.inv_dn, gu->row_norm, tb.hn2};
        const bool f16_out = moe_gate_up_f16_out(gu, I);
        if (int st = launch_moe_gemm(gu->g, wgu, gu_tiled ? gu->tiles : nullptr, gu->tile_bytes, true, tb.xh_gu,
                                     f16_stride(H), tb.inv_gu, tb.perm, k, tb.act, I, I, tb.tile_e, tb.tile_p0,
                                     tb.tile_n, tb.n_tiles, tb.max_tiles, s, f16_out ? &direct : nullptr))
            return st;
        if (!f16_out)
            if (int st = launch_x_to_f16(tb.act, I, I, nullptr, 1, N, tb.xh_dn, f16_stride(I), tb.inv_dn, s)) return st;
        if (int st = launch_moe_gemm(dn->g, wdn, dn->tiles, dn->tile_bytes, false, tb.xh_dn, f16_stride(I),
                                     tb.inv_dn, nullptr, 1, tb.ysl, H, I, tb.tile_e, tb.tile_p0, tb.tile_n,
                                     tb.n_tiles, tb.max_tiles, s))
            return st;
    } else if (moe_mfma_ok(gu, dn, h, H, I)) {
        // decode on MFMA; one token with k <= 2 (out apart from h): gate_up
        // and down in one launch, the combine folded into down
        if (T == 1 && k <= 2 && apart && moe_decode1_ok(gu, dn)) switch (gu->g.type) {
                case LQ_Q6_K: return launch_decode1_t<LQ_Q6_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s);
                case LQ_Q8_0: return launch_decode1_t<LQ_Q8_0>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s);
                default: return launch_decode1_t<LQ_Q4_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s);
            }
        // k <= 2: down adds gate * y onto out (cleared by gate_up) itself,
        // unless out overlaps h (gate_up still reads h)
        float *fold = k <= 2 && apart ? out : nullptr;
        const int st =
            gu->g.type == LQ_Q6_K   ? launch_moe_mfma_t<LQ_Q6_K>(gu, dn, tb, h, H, I, k, slots, fold, topk_w, T, s)
            : gu->g.type == LQ_Q8_0 ? launch_moe_mfma_t<LQ_Q8_0>(gu, dn, tb, h, H, I, k, slots, fold, topk_w, T, s)
                                    : launch_moe_mfma_t<LQ_Q4_K>(gu, dn, tb, h, H, I, k, slots, fold, topk_w, T, s);
        if (st) return st;
        if (fold) return LOCALAI_OK;
    } else {
        if (int st = launch_grouped<true>(gu, tb, h, H, k, slots, T, s)) return st;
        if (int st = launch_grouped<false>(dn, tb, tb.act, I, k, slots, T, s)) return st;
    }
    const bool vec = H % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    const dim3 vgrid((unsigned)((H / 4 + 255) / 256), (unsigned)T);
    if (vec && k == 8)
        hipLaunchKernelGGL(moe_combine_vec_kernel<8>, vgrid, dim3(256), 0, s, tb.ysl, tb.pos, topk_w, (int)H, out);
    else if (vec && k == 4)
        hipLaunchKernelGGL(moe_combine_vec_kernel<4>, vgrid, dim3(256), 0, s, tb.ysl, tb.pos, topk_w, (int)H, out);
    else if (vec && k == 2)
        hipLaunchKernelGGL(moe_combine_vec_kernel<2>, vgrid, dim3(256), 0, s, tb.ysl, tb.pos, topk_w, (int)H, out);
    else
        hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)T), dim3(256), 0, s,
                           tb.ysl, tb.pos, topk_w, k, (int)H, out);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// One of the two expert GEMMs of the prefill path (which = 0: gate_up with
// SiLU*up into the act rows, 1: down into the per-assignment rows), run again
// on the routing tables, f16 rows and act rows that the last launch_moe over
// T tokens left in ws: the measurement of one kernel of the layer alone.
int launch_moe_expert_gemm(const localai_qmat *gu, const localai_qmat *dn, int64_t T, int64_t E, int k, void *ws,
                           int which, hipStream_t s) {
    const int64_t H = gu->g.cols, I = gu->g.rows / 2;
    MoeTables tb = carve(ws, T, E, k, H, I);
    if (tb.tile_w <= 0) return fail(LOCALAI_EARG, "moe expert gemm: fewer tokens than the expert GEMM path takes");
    if (which == 0) {
        const bool tiled = gu->tiles && I % MT_ROWS == 0;
        if (!tiled && !gu->data) return fail(LOCALAI_ESTATE, "moe expert gemm: run the layer once first");
        const MoeF16Out direct{tb.xh_dn, f16_stride(I), tb.inv_dn, gu->row_norm, tb.hn2};
        return launch_moe_gemm(gu->g, tiled ? nullptr : gu->data, tiled ? gu->tiles : nullptr, gu->tile_bytes, true,
                               tb.xh_gu, f16_stride(H), tb.inv_gu, tb.perm, k, tb.act, I, I, tb.tile_e, tb.tile_p0,
                               tb.tile_n, tb.n_tiles, tb.max_tiles, s, moe_gate_up_f16_out(gu, I) ? &direct : nullptr);
    }
    if (!dn->tiles && !dn->data) return fail(LOCALAI_ESTATE, "moe expert gemm: run the layer once first");
    return launch_moe_gemm(dn->g, dn->tiles ? nullptr : dn->data, dn->tiles, dn->tile_bytes, false, tb.xh_dn,
                           f16_stride(I), tb.inv_dn, nullptr, 1, tb.ysl, H, I, tb.tile_e, tb.tile_p0, tb.tile_n,
                           tb.n_tiles, tb.max_tiles, s);
}

// Zeroes the counter block of moe_decode1_kernel (a kernel, not a memset, so
// that the call can be captured in a graph)
__global__ void d1_clear_kernel(uint32_t *__restrict__ sync) {
    for (int i = threadIdx.x; i < D1_WORDS; i += blockDim.x) sync[i] = 0u;
}

// The expert part of the one-token MoE layer from expert indices and weights
// already in device memory (written by a router kernel, e.g. ZAYA's router
// MLP): out = sum_s topk_w[s] * (topk_idx[s] == skip ? h : expert(h)).
int launch_moe_experts1(const float *h, int64_t H, const localai_qmat *gu, const localai_qmat *dn, int k,
                        const int32_t *topk_idx, const float *topk_w, int skip, float *out, void *ws,
                        hipStream_t s) {
    const int64_t I = gu->g.rows / 2, E = gu->g.batch;
    if (!moe_mfma_ok(gu, dn, h, H, I) || !moe_decode1_ok(gu, dn))
        return fail(LOCALAI_ETYPE,
                    "moe experts: Q4_K, Q6_K or Q8_0 experts in the tile form, at most 32 blocks of 256 a row");
    if (out < h + H && h < out + H) return fail(LOCALAI_EARG, "moe experts: out overlaps h");
    MoeTables tb = carve(ws, 1, E, k, H, I);
    hipLaunchKernelGGL(d1_clear_kernel, dim3(1), dim3(256), 0, s, tb.sync);
    LQ_HIP(hipGetLastError());
    switch (gu->g.type) {
        case LQ_Q6_K: return launch_decode1_t<LQ_Q6_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, skip);
        case LQ_Q8_0: return launch_decode1_t<LQ_Q8_0>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, skip);
        default: return launch_decode1_t<LQ_Q4_K>(gu, dn, tb, h, H, E, k, I, topk_idx, topk_w, out, s, skip);
    }
}

}  // namespace lq
