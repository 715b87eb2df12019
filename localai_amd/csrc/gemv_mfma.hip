// Decode matvec on i8 MFMA over the tile form of Q4_K / Q6_K matrices:
// y[r] = sum_c W[r, c] * x[c]. The tile form, the arithmetic and the
// building blocks are described in mfma_core.h; this file holds the repack
// into the tile form, the matvec kernels (one matrix, or several matrices
// with one x in a single launch) and their launch plan.
#include "mfma_core.h"
#include "internal.h"

namespace lq {

constexpr int MT_MAX_JOBS = 8;        // matrices per fused launch (localai_hip_matvec_many)

// Bytes of one matrix's tile form; 0 for types without one (their matvecs
// and GEMMs run on the row planes).
int64_t mt_matrix_bytes(const lq_geom &g) {
    if (g.type != LQ_Q4_K && g.type != LQ_Q6_K && g.type != LQ_Q8_0) return 0;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    return lq_align256(tiles * mt_nsb(g) * mt_block_bytes(g.type));
}

// The decode matvec runs on MFMA for Q4_K / Q6_K up to 72 super-blocks per
// row, and for Q8_0 rows of whole 256-value super-blocks (up to 72 of them),
// the launch plan below; other matrices use gemv.hip.
bool mt_matvec_ok(const lq_geom &g) {
    return ((g.type == LQ_Q4_K || g.type == LQ_Q6_K) && g.nb <= 72) ||
           (g.type == LQ_Q8_0 && g.nb % 8 == 0 && g.nb / 8 <= 72);
}

// GGML <-> tile form, one thread per (matrix, row, super-block); UNPACK
// moves the bytes back to GGML order through the same index expressions.
// Packing: rows past the end of the last tile stay zero (the caller clears
// the buffer).
template <bool UNPACK>
__device__ __forceinline__ void mt_mv(uint8_t *ggml, uint8_t *tile) {
    if (UNPACK) *ggml = *tile;
    else *tile = *ggml;
}

template <bool UNPACK>
__global__ void mt_repack_q4k(lq_geom g, uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int64_t dst_matrix_bytes) {
    const int64_t total = g.batch * g.rows * g.nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * g.nb);
        const int64_t rem = i - e * g.rows * g.nb;
        const int64_t row = rem / g.nb, sb = rem - row * g.nb;
        uint8_t *s = src + e * g.ggml_matrix_bytes + row * g.ggml_row_bytes + sb * 144;
        uint8_t *blk = dst + e * dst_matrix_bytes + ((row / MT_ROWS) * g.nb + sb) * MT_Q4K_BLOCK;
        const int n = (int)(row % MT_ROWS);
        for (int c = 0; c < 4; ++c) {
            const int L = n + 16 * c;
            for (int p = 0; p < 4; ++p)
                for (int b = 0; b < 8; ++b) mt_mv<UNPACK>(&s[16 + 32 * p + 8 * c + b], &blk[(p >> 1) * 1024 + L * 16 + (p & 1) * 8 + b]);
        }
        for (int b = 0; b < 16; ++b) mt_mv<UNPACK>(&s[b], &blk[2048 + n * 16 + b]);
    }
}

// Q6_K tile block, lane L = n + 16c:
//   ql piece h (h = 0, 1) [64][16 B]: ql[64h + 8c ..+7], ql[64h + 32 + 8c ..+7]
//   qh piece [64][16 B]:             qh[8c ..+7],       qh[32 + 8c ..+7]
//   scales [16 rows][16 B] (int8), d [16 rows][2 B]
template <bool UNPACK>
__global__ void mt_repack_q6k(lq_geom g, uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int64_t dst_matrix_bytes) {
    const int64_t total = g.batch * g.rows * g.nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * g.nb);
        const int64_t rem = i - e * g.rows * g.nb;
        const int64_t row = rem / g.nb, sb = rem - row * g.nb;
        uint8_t *s = src + e * g.ggml_matrix_bytes + row * g.ggml_row_bytes + sb * 210;
        uint8_t *blk = dst + e * dst_matrix_bytes + ((row / MT_ROWS) * g.nb + sb) * MT_Q6K_BLOCK;
        const int n = (int)(row % MT_ROWS);
        for (int c = 0; c < 4; ++c) {
            const int L = n + 16 * c;
            for (int h = 0; h < 2; ++h)
                for (int b = 0; b < 8; ++b) {
                    mt_mv<UNPACK>(&s[64 * h + 8 * c + b], &blk[h * 1024 + L * 16 + b]);
                    mt_mv<UNPACK>(&s[64 * h + 32 + 8 * c + b], &blk[h * 1024 + L * 16 + 8 + b]);
                    mt_mv<UNPACK>(&s[128 + 32 * h + 8 * c + b], &blk[2048 + L * 16 + 8 * h + b]);
                }
        }
        for (int b = 0; b < 16; ++b) mt_mv<UNPACK>(&s[192 + b], &blk[3072 + n * 16 + b]);
        mt_mv<UNPACK>(&s[208], &blk[3328 + 2 * n]);
        mt_mv<UNPACK>(&s[209], &blk[3328 + 2 * n + 1]);
    }
}

// Q8_0: one thread per (matrix, row, 256-value block); GGML blocks are
// d (2 B) then 32 int8 quants. Blocks past the row end stay zero.
template <bool UNPACK>
__global__ void mt_repack_q80(lq_geom g, uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int64_t dst_matrix_bytes) {
    const int64_t nsb = mt_nsb(g);
    const int64_t total = g.batch * g.rows * nsb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * nsb);
        const int64_t rem = i - e * g.rows * nsb;
        const int64_t row = rem / nsb, sb = rem - row * nsb;
        uint8_t *srow = src + e * g.ggml_matrix_bytes + row * g.ggml_row_bytes;
        uint8_t *blk = dst + e * dst_matrix_bytes + ((row / MT_ROWS) * nsb + sb) * MT_Q80_BLOCK;
        const int n = (int)(row % MT_ROWS);
        for (int j = 0; j < 8; ++j) {
            const int64_t b = sb * 8 + j;
            if (b >= g.nb) break;
            uint8_t *s = srow + b * 34;
            mt_mv<UNPACK>(&s[0], &blk[4096 + n * 16 + 2 * j]);
            mt_mv<UNPACK>(&s[1], &blk[4096 + n * 16 + 2 * j + 1]);
            for (int c = 0; c < 4; ++c)
                for (int q = 0; q < 8; ++q)
                    mt_mv<UNPACK>(&s[2 + 8 * c + q], &blk[(j >> 1) * 1024 + (n + 16 * c) * 16 + 8 * (j & 1) + q]);
        }
    }
}

// direction 0: GGML -> tile form (the buffer cleared first); 1: tile form -> GGML
static int mt_repack_launch(const lq_geom &g, uint8_t *ggml, uint8_t *tiles, int64_t tile_matrix_bytes, int unpack,
                            hipStream_t s) {
    const int64_t total = g.batch * g.rows * mt_nsb(g);
    if (!unpack) LQ_HIP(hipMemsetAsync(tiles, 0, (size_t)(tile_matrix_bytes * g.batch), s));
    if (total <= 0) return LOCALAI_OK;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
#define MT_R(K)                                                                                                   \
    if (unpack) hipLaunchKernelGGL(K<true>, dim3((unsigned)blocks), dim3(256), 0, s, g, ggml, tiles, tile_matrix_bytes); \
    else hipLaunchKernelGGL(K<false>, dim3((unsigned)blocks), dim3(256), 0, s, g, ggml, tiles, tile_matrix_bytes)
    if (g.type == LQ_Q8_0) { MT_R(mt_repack_q80); }
    else if (g.type == LQ_Q6_K) { MT_R(mt_repack_q6k); }
    else { MT_R(mt_repack_q4k); }
#undef MT_R
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_mt_repack(const lq_geom &g, const uint8_t *ggml, uint8_t *dst, int64_t dst_matrix_bytes,
                     hipStream_t s) {
    return mt_repack_launch(g, const_cast<uint8_t *>(ggml), dst, dst_matrix_bytes, 0, s);
}

int launch_mt_unpack(const lq_geom &g, const uint8_t *tiles, int64_t tile_matrix_bytes, uint8_t *ggml,
                     hipStream_t s) {
    return mt_repack_launch(g, ggml, const_cast<uint8_t *>(tiles), tile_matrix_bytes, 1, s);
}

// The decode step's glue around a matvec (the layer path of
// localai_hip_layer_chain, engine/model.py:229-233 and :181-213):
//   prologue PRO   X:    y = W x
//                  NORM: y = inv * (W x), x = src * w already (the launch
//                        that wrote src also wrote src * w, epilogue RES
//                        with y_next), inv = 1 / sqrt(mean(src^2) + eps)
//                        (engine/model.py:82) from the per-tile partial sums
//                        of squares that launch left in ssq_in; W (x * w)
//                        scaled by inv is the reference's W (x * inv * w)
//                        up to rounding
//   epilogue EPI   Y:    y as it is
//                  RES:  y = res + y (the residual adds, :229, :233); with
//                        ssq_out also the sum of y^2 over each 16-row tile,
//                        with y_next also y_next = y * w_next
//                  ROPE: adjacent-pair RoPE of rows (2j, 2j + 1) of each
//                        head, for jobs < rope_jobs (q and k, :205-210)
//                  SILU: the workgroup's two tiles are tile blk of W (gate)
//                        and tile blk of W2 (up): y = silu(gate) * up (:232)
//                  PAIR: the same two tiles, y = W x and y2 = W2 x
// Every input of the glue is loaded before the weights (loads complete in
// order, so the glue then waits for none of the weight bytes), unconditionally
// at clamped indices (a conditional load is split into waits that hold back
// the loads behind it).

// Partial sums of squares of one vector: MT_SSQ floats, those past the
// vector's tiles zero (its producer writes only its own tiles). Lane l holds
// 4l .. 4l + 3 and 256 + 4l .. 256 + 4l + 3.
struct MtSsq {
    float4 a, b;
};
__device__ __forceinline__ MtSsq mt_load_ssq(const float *__restrict__ p, int lane) {
    const float4 *p4 = reinterpret_cast<const float4 *>(p);
    MtSsq s;
    s.a = p4[lane];
    s.b = p4[64 + lane];
    return s;
}
// 1 / sqrt(sum / n_vals + eps): each lane adds its eight partials in a fixed
// order in fp64, then the 64 lanes in an xor butterfly; every step of it adds
// the same two values in either order, so every lane, wave and workgroup
// gets the same bits
__device__ __forceinline__ float mt_norm_inv(const MtSsq &p, int n_vals, float eps) {
    double s = (((double)p.a.x + (double)p.a.y) + ((double)p.a.z + (double)p.a.w)) +
               (((double)p.b.x + (double)p.b.y) + ((double)p.b.z + (double)p.b.w));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)(s / (double)n_vals), eps)));
}

// RT row tiles of one matrix, workgroup index blk within the matrix (job
// `job` of a fused launch). PIPE: the wave's super-blocks stream through
// two register sets (mt_pass_pipe) instead of being requested all at once
// (long rows, where a wave holds several blocks and their dot products would
// otherwise all wait for the last load).
template <int TYPE, int SPW, int RT, bool PIPE = false, int PRO = MT_PRO_X, int EPI = MT_EPI_Y>
__device__ __forceinline__ void mt_matvec_block(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                int64_t tiles, const float *__restrict__ x,
                                                float *__restrict__ y, int64_t blk, const MtGlue &gl = MtGlue{},
                                                int job = 0) {
    constexpr bool PAIR = EPI == MT_EPI_SILU || EPI == MT_EPI_PAIR;
    static_assert(!PAIR || RT == 2, "paired tiles: one of W, one of W2");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), wv = wave_id(), sb0 = wv * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int i = threadIdx.x;
    // tile t of the workgroup and the row of thread i (i < RT * 16) in it
    auto tile_of = [&](int t) -> int64_t { return PAIR ? blk : blk * RT + t; };
    const int64_t tile = tile_of((i >> 4) & (RT - 1)), row = tile * MT_ROWS + (i & 15);
    const bool mine = i < RT * 16 && tile < tiles && row < rows;
    const int64_t rowc = row < rows ? row : rows - 1;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], x, nb, sb0, lane);   // x first: it is consumed first
    MtSsq ssq;
    if constexpr (PRO == MT_PRO_NORM)
        if (wv == 0) ssq = mt_load_ssq(gl.ssq_in, lane);
    float res = 0.0f, wn = 0.0f, rc = 0.0f, rs = 0.0f;
    if constexpr (EPI == MT_EPI_RES) {
        res = gl.res[rowc];
        if (gl.y_next) wn = gl.w_next[rowc];
    }
    if constexpr (EPI == MT_EPI_ROPE) {
        if (gl.rope_half > 0) {
            int pj = (int)(rowc % gl.head_dim) >> 1;
            pj = pj < gl.rope_half ? pj : gl.rope_half - 1;
            rc = gl.cos[pj];
            rs = gl.sin[pj];
        }
    }
    float inv = 1.0f;
    // run once the weights are requested: the norm factor (wave 0, which
    // writes the results)
    auto prep = [&](const float4 (&in)[SPW], float4 (&out)[SPW]) {
        if constexpr (PRO == MT_PRO_NORM)
            if (wv == 0) inv = mt_norm_inv(ssq, gl.n, gl.eps);
#pragma unroll
        for (int k = 0; k < SPW; ++k) out[k] = in[k];
    };
    float *fin;
    if constexpr (PIPE) {
        static_assert(!PAIR, "paired tiles are for rows of at most 32 super-blocks");
        const uint8_t *tp[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const int64_t tl = tile_of(t) < tiles ? tile_of(t) : tiles - 1;
            tp[t] = Wt + tl * nb * mt_block_bytes(TYPE);
        }
        mt_pass_pipe<TYPE, SPW, RT>(tp, nb, sb0, nsb, xv[0], smem, fin, prep);
    } else {
        MtW<TYPE> w[RT][SPW];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const int64_t tl = tile_of(t) < tiles ? tile_of(t) : tiles - 1;
            const uint8_t *base = (PAIR && t == 1) ? gl.Wt2 : Wt;
            mt_load_tile<TYPE, SPW>(w[t], base + tl * nb * mt_block_bytes(TYPE), nb, sb0, nsb, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
        float4 xp[1][SPW];
        prep(xv[0], xp[0]);
        mt_pass<TYPE, SPW, RT, 1>(w, xp, nsb, smem, fin);
    }
    float v = 0.0f;
    if constexpr (EPI == MT_EPI_SILU) {
        if (i < 16 && tile < tiles && row < rows)
            y[row] = __fmul_rn(silu(__fmul_rn(fin[i], inv)), __fmul_rn(fin[16 + i], inv));
        return;
    }
    if constexpr (EPI == MT_EPI_PAIR) {
        if (mine) (i < 16 ? y : gl.y2)[row] = __fmul_rn(fin[i], inv);
        return;
    }
    if (mine) {
        v = __fmul_rn(fin[i], inv);
        if constexpr (EPI == MT_EPI_RES) v = __fadd_rn(res, v);
        if constexpr (EPI == MT_EPI_ROPE) {
            const int dd = (int)(row % gl.head_dim), pj = dd >> 1;
            if (job < gl.rope_jobs && pj < gl.rope_half) {
                const float other = __fmul_rn(fin[i ^ 1], inv);
                v = (dd & 1) ? __fadd_rn(__fmul_rn(other, rs), __fmul_rn(v, rc))
                             : __fsub_rn(__fmul_rn(v, rc), __fmul_rn(other, rs));
            }
        }
        y[row] = v;
        if constexpr (EPI == MT_EPI_RES)
            if (gl.y_next) gl.y_next[row] = __fmul_rn(v, wn);
    }
    if constexpr (EPI == MT_EPI_RES) {
        // wave 0 (all of its lanes, for the shuffles): the sum of y^2 over
        // each 16-row tile, lanes 16t .. 16t + 15 in an xor butterfly
        if (gl.ssq_out && i < 64) {
            double q = mine ? (double)v * (double)v : 0.0;
#pragma unroll
            for (int m = 8; m >= 1; m >>= 1) q += __shfl_xor(q, m, 64);
            if (i < RT * 16 && (i & 15) == 0 && tile < tiles) gl.ssq_out[tile] = (float)q;
        }
    }
}

// Q4_K workgroups of 1024 threads are held to 64 VGPRs (8 waves per SIMD) so
// that two fit on a CU; the Q6_K body needs more registers than that
template <int TYPE, int SPW, int RT, int MAXT, bool PIPE = false>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(MAXT == 1024 && TYPE == LQ_Q4_K ? 8 : 1)))
void gemv_mfma(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                  int64_t tiles, const float *__restrict__ x,
                                                  float *__restrict__ y) {
    mt_matvec_block<TYPE, SPW, RT, PIPE>(Wt, rows, nb, tiles, x, y, blockIdx.x);
}

// Several matrices with the same K and the same x in one launch: job j owns
// workgroups blk0[j] .. blk0[j + 1] - 1 (uniform branch per workgroup).
struct MtJobs {
    const uint8_t *Wt[MT_MAX_JOBS];
    float *y[MT_MAX_JOBS];
    int64_t rows[MT_MAX_JOBS];
    int64_t blk0[MT_MAX_JOBS + 1];
    int type[MT_MAX_JOBS];
    int n;
};
// Q6 = false: Q4_K jobs only (no Q6_K body compiled in, 64 VGPRs at 1024 threads)
// RT6: row tiles per workgroup of the Q6_K jobs (RT those of the Q4_K jobs)
template <int SPW, int RT, int MAXT, bool Q6, bool PIPE = false, int RT6 = RT>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(MAXT == 1024 && !Q6 ? 8 : 1)))
void gemv_mfma_many(MtJobs jobs, int nb, const float *__restrict__ x) {
    const int64_t b = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < MT_MAX_JOBS; ++i)
        if (i < jobs.n && b >= jobs.blk0[i]) j = i;
    const int64_t tiles = (jobs.rows[j] + MT_ROWS - 1) / MT_ROWS;
    if (Q6 && jobs.type[j] == LQ_Q6_K)
        mt_matvec_block<LQ_Q6_K, SPW, RT6, PIPE>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j], b - jobs.blk0[j]);
    else
        mt_matvec_block<LQ_Q4_K, SPW, RT, PIPE>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j], b - jobs.blk0[j]);
}

// The same kernels with the decode step's glue (MtGlue): one matrix, or
// fused matrices sharing x (job j of the table)
// (64 VGPRs only where a workgroup has 16 waves, SPW = 1)
template <int TYPE, int SPW, int RT, int MAXT, bool PIPE, int PRO, int EPI>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(MAXT == 1024 && TYPE == LQ_Q4_K && SPW == 1 ? 8 : 1)))
void gemv_mfma_glue(const uint8_t *__restrict__ Wt, int64_t rows, int nb, int64_t tiles,
                    const float *__restrict__ x, float *__restrict__ y, MtGlue gl) {
    mt_matvec_block<TYPE, SPW, RT, PIPE, PRO, EPI>(Wt, rows, nb, tiles, x, y, blockIdx.x, gl, 0);
}

// RT6: row tiles per workgroup of the Q6_K jobs (RT those of the Q4_K jobs)
template <int SPW, int RT, int MAXT, bool Q6, bool PIPE, int PRO, int EPI, int RT6 = RT>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(MAXT == 1024 && !Q6 && SPW == 1 ? 8 : 1)))
void gemv_mfma_many_glue(MtJobs jobs, int nb, const float *__restrict__ x, MtGlue gl) {
    const int64_t b = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < MT_MAX_JOBS; ++i)
        if (i < jobs.n && b >= jobs.blk0[i]) j = i;
    const int64_t tiles = (jobs.rows[j] + MT_ROWS - 1) / MT_ROWS;
    if (Q6 && jobs.type[j] == LQ_Q6_K)
        mt_matvec_block<LQ_Q6_K, SPW, RT6, PIPE, PRO, EPI>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j],
                                                           b - jobs.blk0[j], gl, j);
    else
        mt_matvec_block<LQ_Q4_K, SPW, RT, PIPE, PRO, EPI>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j],
                                                          b - jobs.blk0[j], gl, j);
}

// Launch plan: the waves of a workgroup split the super-blocks of one row
// tile (or RT tiles), SPW super-blocks per wave.
//   nb <= 32, >= 768 tiles: SPW = ceil(nb / 16), up to 16 waves, two tiles
//             per workgroup when SPW = 1 (x staged once for both)
//   nb <= 32, fewer tiles:  SPW = ceil(nb / 8), up to 8 waves, one tile per
//             workgroup, so that small matrices still spread over the CUs
//   nb > 32:  SPW = ceil(nb / 8) (5..9), 8 waves, the wave's blocks
//             streamed through two register sets (mt_pass_pipe): Q6_K
//             4096 x 14336 took 12.1 us with all of a wave's blocks requested
//             at once (12 waves x 5) and 11.5 us this way
struct MtPlan {
    int spw, waves, rt;
    bool pipe;
};
static MtPlan mt_plan(int nb, int64_t tiles, bool q6) {
    MtPlan p;
    const bool big = tiles >= 768;
    p.pipe = nb > 32;
    p.spw = nb > 32 ? (nb + 7) / 8 : big ? (nb + 15) / 16 : (nb + 7) / 8;
    p.waves = (nb + p.spw - 1) / p.spw;
    p.rt = (big && p.spw == 1 && !q6) ? 2 : 1;   // two Q6_K tiles need more registers
    return p;
}

#define MT_DISPATCH(L)                                         \
    if (p.pipe) {                                              \
        switch (p.spw) {                                       \
            case 5: L(5, 1, 512, true); break;                 \
            case 6: L(6, 1, 512, true); break;                 \
            case 7: L(7, 1, 512, true); break;                 \
            case 8: L(8, 1, 512, true); break;                 \
            default: L(9, 1, 512, true); break;                \
        }                                                      \
    } else {                                                   \
        switch (p.spw) {                                       \
            case 1: if (p.rt == 2) L(1, 2, 1024, false); else L(1, 1, 1024, false); break; \
            case 2: L(2, 1, 1024, false); break;               \
            case 3: L(3, 1, 768, false); break;                \
            default: L(4, 1, 768, false); break;               \
        }                                                      \
    }

// One vector, many row tiles (the vocabulary head): one workgroup per CU
// (a wave per super-block, rows of up to 16 super-blocks) loops over groups
// of RT tiles, blk, blk + grid, ... . x is staged into LDS and its A operands
// loaded into registers once per workgroup rather than once per tile, and
// the next group's weights are requested before the current group's dot
// products, so each CU streams weights without the gaps between the
// one-tile workgroups of the plain kernel, whose waves each staged x for
// four MFMAs. Dot products and the cross-wave sum are mt_pass's (results
// bit-identical to gemv_mfma's); the wave partials go through two
// alternating LDS buffers, one barrier per group.
template <int TYPE, int RT>
__global__ __launch_bounds__(1024) void gemv_mfma_loop(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                       int64_t tiles, const float *__restrict__ x,
                                                       float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int XB = mt_xbytes(TYPE);
    const int lane = lane_id(), wv = wave_id(), nw = blockDim.x >> 6;   // nw == nb
    const int64_t tile_bytes = (int64_t)nb * mt_block_bytes(TYPE), step = (int64_t)gridDim.x * RT;
    uint8_t *wl = smem + wv * XB;
    float *red = reinterpret_cast<float *>(smem + nw * XB);   // [2][nw][RT][64]
    const uint8_t *wsb = Wt + (int64_t)wv * mt_block_bytes(TYPE);   // the wave's super-block of tile 0
    auto load = [&](MtW<TYPE>(&w)[RT], int64_t t0) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const int64_t tl = t0 + t < tiles ? t0 + t : tiles - 1;
            w[t] = mt_load_w<TYPE>(wsb + tl * tile_bytes, lane);
        }
    };
    const float4 xv = *reinterpret_cast<const float4 *>(x + 256 * wv + 4 * lane);
    MtW<TYPE> wa[RT], wb[RT];
    int64_t t0 = (int64_t)blockIdx.x * RT;
    load(wa, t0);
    __builtin_amdgcn_sched_barrier(0);
    mt_stage<TYPE>(xv, wl, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const MtLane<TYPE> L = mt_lane<TYPE>(lane);
    const MtA<TYPE> a = mt_load_a<TYPE>(wl, L);
    auto group = [&](const MtW<TYPE>(&w)[RT], MtW<TYPE>(&next)[RT], int64_t t0, int buf) {
        // unconditional (past the end: the last tile again, from L2): a
        // conditional request made the compiler's waits for the current set
        // count as if it had not been issued, and wait for it too
        load(next, t0 + step);
        __builtin_amdgcn_sched_barrier(0);
        float *r = red + buf * nw * RT * 64;
#pragma unroll
        for (int t = 0; t < RT; ++t) r[(wv * RT + t) * 64 + lane] = mt_dot<TYPE>(w[t], a, L, 0.0f);
        __syncthreads();
        const int i = threadIdx.x;
        if (i < RT * 16) {
            const int t = i >> 4, n = i & 15;
            float v = 0.0f;
            for (int kk = 0; kk < nw; ++kk) {
                const float *q = r + (kk * RT + t) * 64 + n;
                v += (q[0] + q[16]) + (q[32] + q[48]);
            }
            const int64_t row = (t0 + t) * MT_ROWS + n;
            if (t0 + t < tiles && row < rows) y[row] = v;
        }
    };
    // two copies of the group body, one per register set (the sets alternate)
    while (t0 < tiles) {
        group(wa, wb, t0, 0);
        t0 += step;
        if (t0 >= tiles) break;
        group(wb, wa, t0, 1);
        t0 += step;
    }
}

// Row tiles from which a one-vector matvec of up to 16 super-blocks per row
// runs gemv_mfma_loop (a few groups per CU and more)
constexpr int64_t MT_LOOP_TILES = 2048;
constexpr int MT_LOOP_RT = 2;

int launch_matvec_mfma(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, hipStream_t s) {
    if (!mt_matvec_ok(g)) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K, or Q8_0 with cols % 256 == 0");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)mt_nsb(g);   // 256-value super-blocks per row
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    const bool q6 = g.type == LQ_Q6_K, q8 = g.type == LQ_Q8_0;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    if (nb <= 16 && tiles >= MT_LOOP_TILES) {
        int dev = 0, cus = 0;
        LQ_HIP(hipGetDevice(&dev));
        LQ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        // as many workgroups as CUs, or fewer so that each runs the same count of groups
        const int64_t groups = (tiles + MT_LOOP_RT - 1) / MT_LOOP_RT;
        const int64_t per = (groups + cus - 1) / cus;
        const dim3 lgrid((unsigned)((groups + per - 1) / per)), lblock(64 * nb);
        const size_t llds = (size_t)nb * mt_xbytes(g.type) + (size_t)2 * nb * MT_LOOP_RT * 64 * 4;
        if (q6) hipLaunchKernelGGL((gemv_mfma_loop<LQ_Q6_K, MT_LOOP_RT>), lgrid, lblock, llds, s, Wt, g.rows, nb, tiles, x, y);
        else if (q8) hipLaunchKernelGGL((gemv_mfma_loop<LQ_Q8_0, MT_LOOP_RT>), lgrid, lblock, llds, s, Wt, g.rows, nb, tiles, x, y);
        else hipLaunchKernelGGL((gemv_mfma_loop<LQ_Q4_K, MT_LOOP_RT>), lgrid, lblock, llds, s, Wt, g.rows, nb, tiles, x, y);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
    const MtPlan p = mt_plan(nb, tiles, q6 || q8);   // one tile per workgroup for the larger blocks
    dim3 grid((unsigned)((tiles + p.rt - 1) / p.rt)), block(64 * p.waves);
    const size_t lds = mt_lds_bytes(g.type, p.waves, p.spw, 1, p.rt);
#define MT_L(S, R, M, P)                                                                                        \
    do {                                                                                                        \
        if (q6) hipLaunchKernelGGL((gemv_mfma<LQ_Q6_K, S, R, M, P>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y); \
        else if (q8) hipLaunchKernelGGL((gemv_mfma<LQ_Q8_0, S, R, M, P>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y); \
        else hipLaunchKernelGGL((gemv_mfma<LQ_Q4_K, S, R, M, P>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y);    \
    } while (0)
    MT_DISPATCH(MT_L)
#undef MT_L
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// Several vectors, one matrix: y[t] = W x[t] for t < ntok. The workgroup's
// row tiles are loaded into registers once (every block of the wave at
// once) and each vector goes through the single-vector arithmetic of
// mt_pass in turn (so y[t] is bit-identical to a one-vector call on x[t]);
// the next vector's x is requested before the current one is summed. The
// weights are read from HBM once per call however many vectors there are.
template <int TYPE, int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_tok(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                      int64_t tiles, const float *__restrict__ x, int64_t ldx,
                                                      float *__restrict__ y, int64_t ldy, int ntok) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), wv = wave_id(), sb0 = wv * SPW, nsb = mt_nsb(nb, sb0, SPW);
    const int64_t blk = blockIdx.x;
    const int i = threadIdx.x;
    const int64_t tile = blk * RT + ((i >> 4) & (RT - 1)), row = tile * MT_ROWS + (i & 15);
    const bool mine = i < RT * 16 && tile < tiles && row < rows;
    float4 xv[1][SPW];
    mt_load_x<SPW>(xv[0], x, nb, sb0, lane);
    MtW<TYPE> w[RT][SPW];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t tl = blk * RT + t < tiles ? blk * RT + t : tiles - 1;
        mt_load_tile<TYPE, SPW>(w[t], Wt + tl * nb * mt_block_bytes(TYPE), nb, sb0, nsb, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int t = 0; t < ntok; ++t) {
        float4 xn[SPW];
        mt_load_x<SPW>(xn, x + (int64_t)(t + 1 < ntok ? t + 1 : t) * ldx, nb, sb0, lane);
        float *fin;
        mt_pass<TYPE, SPW, RT, 1>(w, xv, nsb, smem, fin);
        if (mine) y[(int64_t)t * ldy + row] = fin[i];
#pragma unroll
        for (int k = 0; k < SPW; ++k) xv[0][k] = xn[k];
    }
}

int launch_matvec_mfma_tok(const lq_geom &g, const uint8_t *Wt, const float *x, int64_t ldx, float *y, int64_t ldy,
                           int ntok, hipStream_t s) {
    if (!mt_matvec_ok(g)) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K, or Q8_0 with cols % 256 == 0");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || ldx % 4)
        return fail(LOCALAI_EARG, "mfma matvec: x rows must be 16-byte aligned");
    if (ntok < 1) return LOCALAI_OK;
    const int nb = (int)mt_nsb(g);
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    const bool q6 = g.type == LQ_Q6_K, q8 = g.type == LQ_Q8_0;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    // up to 32 super-blocks: up to 16 waves (SPW = ceil(nb / 16)), two Q4_K
    // tiles per workgroup where one super-block per wave leaves room, as in
    // the one-vector plan; longer rows: 8 waves of ceil(nb / 8) blocks (up to
    // 9 for K <= 18432), which fit in registers only below 16 waves
    const int spw = nb <= 32 ? (nb + 15) / 16 : (nb + 7) / 8, waves = (nb + spw - 1) / spw;
    const int rt = spw == 1 && tiles >= 768 && !q6 ? 2 : 1;
    dim3 grid((unsigned)((tiles + rt - 1) / rt)), block(64 * waves);
    const size_t lds = mt_lds_bytes(g.type, waves, spw, 1, rt);
#define MT_T(S, R, M)                                                                                          \
    do {                                                                                                       \
        if (q6) hipLaunchKernelGGL((gemv_mfma_tok<LQ_Q6_K, S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, \
                                   ldx, y, ldy, ntok);                                                         \
        else if (q8) hipLaunchKernelGGL((gemv_mfma_tok<LQ_Q8_0, S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, \
                                        x, ldx, y, ldy, ntok);                                                 \
        else hipLaunchKernelGGL((gemv_mfma_tok<LQ_Q4_K, S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, ldx, \
                                y, ldy, ntok);                                                                 \
    } while (0)
    switch (spw) {
        case 1: if (rt == 2) MT_T(1, 2, 1024); else MT_T(1, 1, 1024); break;
        case 2: MT_T(2, 1, 1024); break;
        case 5: MT_T(5, 1, 512); break;
        case 6: MT_T(6, 1, 512); break;
        case 7: MT_T(7, 1, 512); break;
        case 8: MT_T(8, 1, 512); break;
        default: MT_T(9, 1, 512); break;
    }
#undef MT_T
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_matvec_mfma_many(int n, const lq_geom *const *g, const uint8_t *const *Wt, const float *x,
                            float *const *y, hipStream_t s) {
    if (n < 1 || n > MT_MAX_JOBS) return fail(LOCALAI_EARG, "mfma matvec: 1..8 matrices per fused launch");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g[0]->nb;
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    int64_t total_tiles = 0;
    bool any_q6 = false;
    for (int j = 0; j < n; ++j) {
        if (g[j]->type != LQ_Q4_K && g[j]->type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
        if (g[j]->nb != nb) return fail(LOCALAI_EARG, "mfma matvec: fused matrices need the same cols");
        total_tiles += (g[j]->rows + MT_ROWS - 1) / MT_ROWS;
        any_q6 |= g[j]->type == LQ_Q6_K;
    }
    const MtPlan p = mt_plan(nb, total_tiles, any_q6);
    if (n == 2 && !any_q6 && p.spw == 1 && p.rt == 2 && g[0]->rows == g[1]->rows) {
        // two Q4_K matrices of one shape (gate and up): a workgroup takes
        // tile i of each
        const int64_t tiles = (g[0]->rows + MT_ROWS - 1) / MT_ROWS;
        MtGlue gl{};
        gl.Wt2 = Wt[1];
        gl.y2 = y[1];
        hipLaunchKernelGGL((gemv_mfma_glue<LQ_Q4_K, 1, 2, 1024, false, MT_PRO_X, MT_EPI_PAIR>), dim3((unsigned)tiles),
                           dim3(64 * p.waves), mt_lds_bytes(LQ_Q4_K, p.waves, 1, 1, 2), s, Wt[0], g[0]->rows, nb, tiles,
                           x, y[0], gl);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
    // mixed Q4_K / Q6_K groups of the small plan (q/k/v): the Q4_K jobs take
    // two tiles per workgroup, so each wave's staged x serves two tiles
    const bool split = any_q6 && !p.pipe && p.spw == 2 && p.rt == 1;
    MtJobs jobs = {};
    jobs.n = n;
    int64_t b = 0;
    for (int j = 0; j < n; ++j) {
        jobs.Wt[j] = Wt[j];
        jobs.y[j] = y[j];
        jobs.rows[j] = g[j]->rows;
        jobs.type[j] = g[j]->type;
        jobs.blk0[j] = b;
        const int rt = split && g[j]->type == LQ_Q4_K ? 2 : p.rt;
        b += ((g[j]->rows + MT_ROWS - 1) / MT_ROWS + rt - 1) / rt;
    }
    for (int j = n; j <= MT_MAX_JOBS; ++j) jobs.blk0[j] = b;
    dim3 grid((unsigned)b), block(64 * p.waves);
    const size_t lds = mt_lds_bytes(any_q6 ? LQ_Q6_K : LQ_Q4_K, p.waves, p.spw, 1, split ? 2 : p.rt);
    if (split) {
        hipLaunchKernelGGL((gemv_mfma_many<2, 2, 1024, true, false, 1>), grid, block, lds, s, jobs, nb, x);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
#define MT_L(S, R, M, P)                                                                        \
    do {                                                                                        \
        if (any_q6) hipLaunchKernelGGL((gemv_mfma_many<S, R, M, true, P>), grid, block, lds, s, jobs, nb, x);  \
        else hipLaunchKernelGGL((gemv_mfma_many<S, R, M, false, P>), grid, block, lds, s, jobs, nb, x);        \
    } while (0)
    MT_DISPATCH(MT_L)
#undef MT_L
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_matvec_mfma_glue(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, int pro, int epi,
                            const MtGlue &gl, hipStream_t s) {
    if (g.type != LQ_Q4_K && g.type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g.nb;
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    const bool q6 = g.type == LQ_Q6_K;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    MtPlan p = mt_plan(nb, tiles, q6);
    if (epi == MT_EPI_SILU) {
        // gate tile i and up tile i per workgroup, up to 16 waves
        if (nb > 32 || pro != MT_PRO_NORM || !gl.Wt2)
            return fail(LOCALAI_ETYPE, "mfma matvec: paired gate / up tiles need rows of at most 8192 values");
        p.spw = (nb + 15) / 16;
        p.waves = (nb + p.spw - 1) / p.spw;
        p.rt = 2;
        p.pipe = false;
    }
    if (pro == MT_PRO_NORM && (nb > 32 || (reinterpret_cast<uintptr_t>(gl.ssq_in) & 15)))
        return fail(LOCALAI_ETYPE, "mfma matvec: the norm needs rows of at most 8192 values");
    const dim3 grid((unsigned)(epi == MT_EPI_SILU ? tiles : (tiles + p.rt - 1) / p.rt)), block(64 * p.waves);
    const size_t lds = mt_lds_bytes(g.type, p.waves, p.spw, 1, p.rt);
#define MT_L(S, R, M, P)                                                                                    \
    do {                                                                                                    \
        if (q6) hipLaunchKernelGGL((gemv_mfma_glue<LQ_Q6_K, S, R, M, P, PRO_, EPI_>), grid, block, lds, s, Wt, \
                                   g.rows, nb, tiles, x, y, gl);                                            \
        else hipLaunchKernelGGL((gemv_mfma_glue<LQ_Q4_K, S, R, M, P, PRO_, EPI_>), grid, block, lds, s, Wt,    \
                                g.rows, nb, tiles, x, y, gl);                                               \
    } while (0)
    if (pro == MT_PRO_X && epi == MT_EPI_RES) {
        constexpr int PRO_ = MT_PRO_X, EPI_ = MT_EPI_RES;
        MT_DISPATCH(MT_L)
    } else if (pro == MT_PRO_NORM && epi == MT_EPI_SILU) {
        constexpr int PRO_ = MT_PRO_NORM, EPI_ = MT_EPI_SILU;
        if (p.spw == 1) MT_L(1, 2, 1024, false);
        else MT_L(2, 2, 1024, false);
    } else {
        return fail(LOCALAI_ETYPE, "mfma matvec: no kernel for this prologue / epilogue");
    }
#undef MT_L
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_matvec_mfma_many_glue(int n, const lq_geom *const *g, const uint8_t *const *Wt, const float *x,
                                 float *const *y, int pro, int epi, const MtGlue &gl, hipStream_t s) {
    if (n < 1 || n > MT_MAX_JOBS) return fail(LOCALAI_EARG, "mfma matvec: 1..8 matrices per fused launch");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g[0]->nb;
    if (nb > 32 || pro != MT_PRO_NORM || (reinterpret_cast<uintptr_t>(gl.ssq_in) & 15))
        return fail(LOCALAI_ETYPE, "mfma matvec: the norm needs rows of at most 8192 values");
    int64_t total_tiles = 0;
    bool any_q6 = false;
    for (int j = 0; j < n; ++j) {
        if (g[j]->type != LQ_Q4_K && g[j]->type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
        if (g[j]->nb != nb) return fail(LOCALAI_EARG, "mfma matvec: fused matrices need the same cols");
        total_tiles += (g[j]->rows + MT_ROWS - 1) / MT_ROWS;
        any_q6 |= g[j]->type == LQ_Q6_K;
    }
    const MtPlan p = mt_plan(nb, total_tiles, any_q6);
    // mixed Q4_K / Q6_K groups of the small plan (q/k/v): the Q4_K jobs take
    // two tiles per workgroup, so each wave's staged x serves two tiles
    const bool split = any_q6 && !p.pipe && p.spw == 2 && p.rt == 1;
    MtJobs jobs = {};
    jobs.n = n;
    int64_t b = 0;
    for (int j = 0; j < n; ++j) {
        jobs.Wt[j] = Wt[j];
        jobs.y[j] = y[j];
        jobs.rows[j] = g[j]->rows;
        jobs.type[j] = g[j]->type;
        jobs.blk0[j] = b;
        const int rt = split && g[j]->type == LQ_Q4_K ? 2 : p.rt;
        b += ((g[j]->rows + MT_ROWS - 1) / MT_ROWS + rt - 1) / rt;
    }
    for (int j = n; j <= MT_MAX_JOBS; ++j) jobs.blk0[j] = b;
    dim3 grid((unsigned)b), block(64 * p.waves);
    const size_t lds = mt_lds_bytes(any_q6 ? LQ_Q6_K : LQ_Q4_K, p.waves, p.spw, 1, split ? 2 : p.rt);
    if (split) {
        if (epi == MT_EPI_Y)
            hipLaunchKernelGGL((gemv_mfma_many_glue<2, 2, 1024, true, false, MT_PRO_NORM, MT_EPI_Y, 1>), grid, block,
                               lds, s, jobs, nb, x, gl);
        else if (epi == MT_EPI_ROPE)
            hipLaunchKernelGGL((gemv_mfma_many_glue<2, 2, 1024, true, false, MT_PRO_NORM, MT_EPI_ROPE, 1>), grid,
                               block, lds, s, jobs, nb, x, gl);
        else
            return fail(LOCALAI_ETYPE, "mfma matvec: no kernel for this prologue / epilogue");
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
#define MT_L(S, R, M, P)                                                                                    \
    do {                                                                                                    \
        if constexpr (!P) {                                                                                 \
            if (any_q6) hipLaunchKernelGGL((gemv_mfma_many_glue<S, R, M, true, P, PRO_, EPI_>), grid, block, lds, s, \
                                           jobs, nb, x, gl);                                                \
            else hipLaunchKernelGGL((gemv_mfma_many_glue<S, R, M, false, P, PRO_, EPI_>), grid, block, lds, s,  \
                                    jobs, nb, x, gl);                                                       \
        }                                                                                                   \
    } while (0)
    if (epi == MT_EPI_Y) {
        constexpr int PRO_ = MT_PRO_NORM, EPI_ = MT_EPI_Y;
        MT_DISPATCH(MT_L)
    } else if (epi == MT_EPI_ROPE) {
        constexpr int PRO_ = MT_PRO_NORM, EPI_ = MT_EPI_ROPE;
        MT_DISPATCH(MT_L)
    } else {
        return fail(LOCALAI_ETYPE, "mfma matvec: no kernel for this prologue / epilogue");
    }
#undef MT_L
#undef MT_DISPATCH
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
