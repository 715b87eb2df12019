// Prefill matmul on MFMA: Y[t, r] = sum_c W[r, c] * X[t, c] for many tokens.
//
// Counterpart of decoded_matmul_row / localai_*_matmul
// (engine/native_quant.cpp:444-531, :744-768): the reference decodes each row
// exactly to fp32 and runs fp32 FMAs over the tokens. Here weights are decoded
// exactly (the per-type formulas of the dequant kernels), rounded once to f16
// and multiplied with v_mfma_f32_16x16x32_f16 in fp32 accumulation.
//
// Activations are converted once per call (x_to_f16): each token row is scaled
// by a power of two so that its largest magnitude lies in [2^14, 2^15)
// (exact), rounded to f16, and the output is scaled back by the inverse power.
// f16 (11 significant bits) rather than bf16 (8) keeps the normwise error near
// 2^-12. The rows are stored row-major, or (for the CU-tile kernel) in MFMA
// operand order, 1 KB per 16 tokens x 32 values.
//
// Three kernels:
//   gemm_kernel       any type from the GGML bytes: a workgroup decodes a
//                     128-row weight tile into LDS per 128-value step and 4
//                     waves multiply it with 128 tokens (also the MoE expert
//                     tiles of moe.hip);
//   gemm_tile_kernel  Q4_K / Q6_K / Q8_0 from the tile form (mfma_core.h):
//                     each wave decodes its own two 16-row tiles into B
//                     operands in registers, x is staged in LDS
//                     (global_load_lds), dense and MoE;
//   gemm_cu_q80_kernel dense Q8_0 with 256 tokens or more: one 224-row x
//                     128-token tile per CU, sized to what L2 can feed a CU
//                     (its own section below).
#include <type_traits>

#include "f16rows.h"
#include "gemv_core.h"
#include "internal.h"
#include "mfma_core.h"

namespace lq {

typedef _Float16 lq_h8 __attribute__((ext_vector_type(8)));

constexpr int GM_BM = 128;             // weight rows per workgroup
constexpr int GM_BN = 128;             // tokens per workgroup (dense)
constexpr int GM_MOE_BN = 64;          // tokens per workgroup (MoE expert tiles)
constexpr int GM_BK = 128;             // K values per step (two 64-value units)
constexpr int GM_LD = GM_BK + 8;       // LDS row stride in halves (272 B: 16 lanes of a
                                       // 16-byte read hit 16 distinct bank groups)

// ---------------------------------------------------------------- activations

// One wave per token row, four rows per workgroup (x_to_f16_row, f16rows.h).
template <int NG>
__global__ __launch_bounds__(256) void x_to_f16_kernel(const float *__restrict__ X, int64_t ldx, int cols,
                                                       const int32_t *__restrict__ rows_map, int k, int64_t ntok,
                                                       _Float16 *__restrict__ Xh, int ldh,
                                                       float *__restrict__ inv, int vec, int tiled, int64_t ntok_pad,
                                                       float *__restrict__ nrm2) {
    const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave_id();
    x_to_f16_row<NG>(t, X, ldx, cols, rows_map, k, ntok, Xh, ldh, inv, vec, tiled, ntok_pad, nrm2);
}

// ---------------------------------------------------------------- weights

// Exact fp32 values of unit u in unit order (the order of gemv_core.h's x
// windows); the same formulas as engine/dequant.py:62-165.
template <int T>
__device__ __forceinline__ void dequant_unit(const UnitW &w, int u, float *out) {
    if constexpr (T == LQ_Q4_K || T == LQ_Q5_K) {
        const int p = u & 3;
        uint32_t sc0, sc1, mn0, mn1;
        kq_pair(w.h0, p, sc0, sc1, mn0, mn1);
        const float d = f16_to_f32(w.h0.x), dmin = f16_to_f32(w.h0.x >> 16);
        const float a0 = d * (float)sc0, a1 = d * (float)sc1;
        const float b0 = dmin * (float)mn0, b1 = dmin * (float)mn1;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint32_t byte = (u4_get(j < 16 ? w.q0 : w.q1, (j & 15) >> 2) >> (8 * (j & 3))) & 0xFFu;
            uint32_t lo = byte & 15u, hi = byte >> 4;
            if constexpr (T == LQ_Q5_K) {
                const uint32_t qh = (u4_get(j < 16 ? w.h1 : w.q2, (j & 15) >> 2) >> (8 * (j & 3))) & 0xFFu;
                lo |= ((qh >> (2 * p)) & 1u) << 4;
                hi |= ((qh >> (2 * p + 1)) & 1u) << 4;
            }
            out[j] = __builtin_fmaf(a0, (float)lo, -b0);
            out[32 + j] = __builtin_fmaf(a1, (float)hi, -b1);
        }
    } else if constexpr (T == LQ_Q6_K) {
        const float d = f16_to_f32(w.d);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float dc = d * (float)(int8_t)(w.sc >> (8 * c));
            const uint4 ql = (c & 1) ? w.q1 : w.q0;
            const uint32_t sh = (c >> 1) * 4, hs = 2 * c;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t qb = (u4_get(ql, e >> 2) >> (8 * (e & 3) + sh)) & 15u;
                const uint32_t hb = (u4_get(w.h0, e >> 2) >> (8 * (e & 3) + hs)) & 3u;
                out[16 * c + e] = dc * (float)((int)(qb | (hb << 4)) - 32);
            }
        }
    } else if constexpr (T == LQ_Q8_0) {
        const float d0 = f16_to_f32(w.sc), d1 = f16_to_f32(w.sc >> 16);
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            const uint4 q = j < 16 ? w.q0 : j < 32 ? w.q1 : j < 48 ? w.q2 : w.q3;
            const int v = (int)(int8_t)(u4_get(q, (j & 15) >> 2) >> (8 * (j & 3)));
            out[j] = (j < 32 ? d0 : d1) * (float)v;
        }
    } else {   // Q4_0
        const float d0 = f16_to_f32(w.sc), d1 = f16_to_f32(w.sc >> 16);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint4 q = j < 16 ? w.q0 : w.q1;
            const uint32_t byte = (u4_get(q, (j & 15) >> 2) >> (8 * (j & 3))) & 0xFFu;
            const float d = j < 16 ? d0 : d1;
            out[2 * (j & ~15) + (j & 15)] = d * (float)((int)(byte & 15u) - 8);
            out[2 * (j & ~15) + 16 + (j & 15)] = d * (float)((int)(byte >> 4) - 8);
        }
    }
}

// Position inside the 128-value step window of value j (unit order) of unit u.
template <int T>
__device__ __forceinline__ int window_pos(int u, int j) {
    if constexpr (T == LQ_Q6_K) return 32 * (j >> 4) + 16 * (u & 1) + (j & 15);
    else return 64 * (u & 1) + j;
}

typedef _Float16 lq_h2 __attribute__((ext_vector_type(2)));

// Bytes 0, 1 (lo) or 2, 3 (hi) of w below the exponent byte 0x64: two f16
// values 1024 + byte (one v_perm_b32; selector bytes 0..3 pick w's bytes,
// 4 picks the first byte of 0x64646464).
__device__ __forceinline__ uint32_t f16_bytes_lo(uint32_t w) {
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
}
__device__ __forceinline__ uint32_t f16_bytes_hi(uint32_t w) {
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
}

// Q8_0 weights straight to f16 pairs: byte q + 128 under the f16 exponent of
// 1024 reads as 1152 + q (exact), minus 1152 gives q exactly, and one f16
// multiply by d rounds d * q once (the same value as rounding the exact fp32
// product). Four int8 quants in `w` -> two f16 pairs.
__device__ __forceinline__ void q8_pairs(uint32_t w, lq_h2 d2, uint32_t &lo, uint32_t &hi) {
    const uint32_t b = w ^ 0x80808080u;
    const uint32_t l = f16_bytes_lo(b), h = f16_bytes_hi(b);
    const lq_h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(lq_h2, l) - off) * d2);
    hi = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(lq_h2, h) - off) * d2);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// ---------------------------------------------------------------- GEMM

enum { GM_DENSE = 0, GM_MOE_GATE_UP = 1, GM_MOE_DOWN = 2 };

// Dense: token tile blockIdx.y of Xh [ntok, ldh]; Y[t * y_ts + r * y_rs].
// MoE: work tile blockIdx.y of the expert tile list (expert, first row of
// the expert-major Xh, valid rows); gate_up writes silu(g) * u to
// Y[p * y_ts + r] for r < inter, down writes Y[p * y_ts + r].
struct GemmArgs {
    lq_geom g;
    const uint8_t *W;          // dense: the matrix; MoE: expert 0 of the [E, rows, cols] handle
    const _Float16 *Xh;        // f16 rows, stride ldh (zero past cols)
    int ldh;
    const float *inv;          // per Xh row output scale
    int64_t ntok;
    float *Y;
    int64_t y_ts, y_rs;
    const int32_t *tile_e, *tile_p0, *tile_n, *n_tiles;
    int64_t inter;
    const uint8_t *Wt;         // tile form (mfma_core.h) or null; MoE: expert 0
    int64_t wt_bytes;          // tile-form bytes per matrix
    const int32_t *rows_map;   // null, or: token p reads Xh / inv row rows_map[p] / rows_k
    int rows_k;
    // MoE gate_up on the tile form, f16 output (Yh not null): SiLU * up of
    // token p goes to Yh row p (stride ldy) times 2^s, inv_out[p] = 2^-s, s
    // from the bound 4 |gate rows| |up rows| |h row|^2 (wnorm: the expert
    // handle's row_norm, xnorm2: sum of squares per Xh row)
    _Float16 *Yh;
    int64_t ldy;
    float *inv_out;
    const float *wnorm, *xnorm2;
};

// Xh / inv row of token position p
__device__ __forceinline__ int64_t gemm_xrow(const GemmArgs &a, int64_t p) {
    return a.rows_map ? (int64_t)(a.rows_map[p] / a.rows_k) : p;
}

template <int T, int BN, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    constexpr int NI = BN / 32;            // 16-token MFMA tiles per wave (waves split tokens in 2)
    __shared__ __attribute__((aligned(16))) _Float16 Ws[GM_BM * GM_LD];
    __shared__ __attribute__((aligned(16))) _Float16 Xs[BN * GM_LD];
    const lq_geom &g = a.g;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    // token tile
    const uint8_t *W = a.W;
    int64_t p0;
    int tn;
    int64_t rtile;
    if constexpr (MODE == GM_DENSE) {
        // 1-D grid, padded to a multiple of 8. Workgroups are dispatched to the
        // 8 XCDs round-robin (id % 8); workgroup id -> logical index
        // xcd * per + id / 8 walks the row tiles of one token tile per XCD, so
        // each XCD's L2 holds one activation tile while the weights stream.
        const int id = blockIdx.x, per = gridDim.x / 8;
        const int L = (id % 8) * per + id / 8;
        const int nrt = (int)((g.rows + GM_BM - 1) / GM_BM);
        const int64_t ntt = (a.ntok + BN - 1) / BN;
        if (L >= nrt * ntt) return;
        rtile = L % nrt;
        p0 = (int64_t)(L / nrt) * BN;
        tn = (int)(a.ntok - p0 < BN ? a.ntok - p0 : BN);
    } else {
        rtile = blockIdx.x;
        const int tile = blockIdx.y;
        if (tile >= a.n_tiles[0]) return;
        W += (int64_t)a.tile_e[tile] * g.matrix_bytes;
        p0 = a.tile_p0[tile];
        tn = a.tile_n[tile];
    }
    // weight rows of this tile: q -> matrix row (or -1 when past the end)
    const int64_t r0 = rtile * (MODE == GM_MOE_GATE_UP ? GM_BM / 2 : GM_BM);
    auto row_of = [&](int q) -> int64_t {
        if constexpr (MODE == GM_MOE_GATE_UP) {
            // wave row block rb = q / 64, MFMA tile j = (q % 64) / 16: j < 2 gate, j >= 2 up,
            // so a lane holds the gate and up sums of the same row in tiles j and j + 2
            const int rb = q >> 6, j = (q >> 4) & 3, rr = q & 15;
            const int64_t r = r0 + 32 * rb + 16 * (j & 1) + rr;
            return r < a.inter ? r + (j >> 1) * a.inter : -1;
        } else {
            return r0 + q < g.rows ? r0 + q : -1;
        }
    };
    const int U = (int)g.nu, steps = (U + 1) / 2;
    const int lr = tid >> 1, lh = tid & 1;
    int64_t wrow = row_of(lr);
    wrow = wrow < 0 ? 0 : wrow;
    // activation loader: BN rows x 128 values, 256 threads
    constexpr int XT = 256 / BN;              // threads per token row (2 or 4 or 8)
    constexpr int XV = 128 / XT;              // halves per thread
    const int xr = tid / XT, xp = tid % XT;
    const int64_t xrow = gemm_xrow(a, p0 + (xr < tn ? xr : 0));
    const _Float16 *xsrc = a.Xh + xrow * a.ldh + XV * xp;

    UnitW wreg;
    uint4 xreg[XV / 8];
    auto load = [&](int step) {
        const int u = 2 * step + lh;
        const int uc = u < U ? u : U - 1;
        const int c0 = uc & ~63;
        const int C = U - c0 < 64 ? U - c0 : 64;
        wreg = load_unit_w<T>(W, g, wrow, uc, C);
        const uint4 *xp4 = reinterpret_cast<const uint4 *>(xsrc + (int64_t)step * GM_BK);
#pragma unroll
        for (int i = 0; i < XV / 8; ++i) xreg[i] = xp4[i];
    };
    auto store = [&](int step) {
        const int u = 2 * step + lh;
        const bool valid = u < U;
        _Float16 *wd = Ws + lr * GM_LD;
        if constexpr (T == LQ_Q8_0) {
            const uint32_t dm = valid ? 0xFFFFFFFFu : 0u;
            const lq_h2 d0 = __builtin_bit_cast(lq_h2, ((wreg.sc & 0xFFFFu) * 0x10001u) & dm);
            const lq_h2 d1 = __builtin_bit_cast(lq_h2, ((wreg.sc >> 16) * 0x10001u) & dm);
            const uint4 qs[4] = {wreg.q0, wreg.q1, wreg.q2, wreg.q3};
#pragma unroll
            for (int c = 0; c < 8; ++c) {      // 8 values per 16-byte LDS write
                const uint4 q = qs[c >> 1];
                const lq_h2 d2 = c < 4 ? d0 : d1;
                uint4 p;
                q8_pairs(u4_get(q, 2 * (c & 1)), d2, p.x, p.y);
                q8_pairs(u4_get(q, 2 * (c & 1) + 1), d2, p.z, p.w);
                *reinterpret_cast<uint4 *>(wd + 64 * (u & 1) + 8 * c) = p;
            }
        } else {
            float v[64];
            dequant_unit<T>(wreg, u < U ? u : U - 1, v);
#pragma unroll
            for (int j = 0; j < 64; j += 8) {
                uint4 p;
                p.x = valid ? pack_h2(v[j + 0], v[j + 1]) : 0u;
                p.y = valid ? pack_h2(v[j + 2], v[j + 3]) : 0u;
                p.z = valid ? pack_h2(v[j + 4], v[j + 5]) : 0u;
                p.w = valid ? pack_h2(v[j + 6], v[j + 7]) : 0u;
                *reinterpret_cast<uint4 *>(wd + window_pos<T>(u, j)) = p;
            }
        }
        uint4 *xd = reinterpret_cast<uint4 *>(Xs + xr * GM_LD + XV * xp);
#pragma unroll
        for (int i = 0; i < XV / 8; ++i) xd[i] = xreg[i];
    };

    lq_f4 acc[NI][4];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = lq_f4{0.0f, 0.0f, 0.0f, 0.0f};

    const int tb = wave >> 1, rb = wave & 1;
    const int fr = lane & 15, fk = 8 * (lane >> 4);
    load(0);
    for (int s = 0; s < steps; ++s) {
        store(s);
        __syncthreads();
        if (s + 1 < steps) load(s + 1);
#pragma unroll
        for (int kk = 0; kk < GM_BK / 32; ++kk) {
            lq_h8 av[NI], bv[4];
#pragma unroll
            for (int i = 0; i < NI; ++i)
                av[i] = *reinterpret_cast<const lq_h8 *>(Xs + ((BN / 2) * tb + 16 * i + fr) * GM_LD + 32 * kk + fk);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bv[j] = *reinterpret_cast<const lq_h8 *>(Ws + (64 * rb + 16 * j + fr) * GM_LD + 32 * kk + fk);
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D[m][n]: lane holds tokens 4 * (lane / 16) + v of token tile i, row lane % 16 of row tile j
#pragma unroll
    for (int i = 0; i < NI; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int lt = (BN / 2) * tb + 16 * i + 4 * (lane >> 4) + v;
            if (lt >= tn) continue;
            const int64_t p = p0 + lt;
            const float sc = a.inv[gemm_xrow(a, p)];
            if constexpr (MODE == GM_MOE_GATE_UP) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t r = r0 + 32 * rb + 16 * j + fr;
                    if (r < a.inter) {
                        const float gv = acc[i][j][v] * sc, uv = acc[i][j + 2][v] * sc;
                        a.Y[p * a.y_ts + r] = silu(gv) * uv;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t r = r0 + 64 * rb + 16 * j + fr;
                    if (r < g.rows) a.Y[p * a.y_ts + r * a.y_rs] = acc[i][j][v] * sc;
                }
            }
        }
    }
}

// --------------------------------------------------- GEMM on the tile form
// Q4_K / Q6_K / Q8_0 handles carry the tile form (mfma_core.h). For a 32-value
// slice of a 256-value block, the 8 quants that lane l (weight row l % 16,
// k = 8 (l / 16) .. + 7) holds in its 16-byte slice are exactly that lane's
// part of the B operand of v_mfma_f32_16x16x32_f16. So a wave decodes its own
// weight rows straight into B registers -- each weight value once per
// workgroup, exactly in fp32 (or, for Q8_0, exactly as 1152 + q in f16 times
// d), rounded once to f16 -- and only the f16 activations (A operands) go
// through LDS, double-buffered and shared by the 4 waves.
//
// Workgroup: 4 waves x 2 row tiles (128 weight rows; for gate_up 64 gate rows
// and the 64 matching up rows) x BN tokens, 128 K values per step.

// Workgroup barrier without the fence of __syncthreads, whose wait for every
// outstanding LDS read would stall on the next step's operand prefetch. What
// crosses it is ordered by hand: each wave waits (vmcnt) for its own copies
// into the ring before arriving, and every read of a ring slot has been
// consumed by an MFMA (lgkmcnt wait) before the barrier that precedes the
// slot's refill. The memory clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void cu_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 1 KB from global memory (16 bytes per lane) into LDS at the wave-uniform
// byte address lds (lane i's bytes at lds + 16 i), through M0, which it saves
// and restores
__device__ __forceinline__ void cu_dma(const void *src, uint32_t lds) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(src), "s"(lds)
                 : "memory");
}
constexpr int GT_WROWS = 128;          // weight rows per workgroup (dense, 4 waves)
constexpr int GM_MOE_NW = 8;           // waves per workgroup of the expert tile GEMMs

template <int T> struct GtRaw;
template <> struct GtRaw<LQ_Q4_K> { uint4 qs, hd; };
template <> struct GtRaw<LQ_Q6_K> { uint4 ql, qh, sc; uint32_t d; };
template <> struct GtRaw<LQ_Q8_0> { uint4 p0, p1, dd; };

// weights of half `half` (values 128 half .. + 127) of one 256-value block
template <int T>
__device__ __forceinline__ GtRaw<T> gt_load(const uint8_t *blk, int half, int lane) {
    GtRaw<T> r;
    const int n = lane & 15;
    if constexpr (T == LQ_Q4_K) {
        r.qs = ld16(blk + half * 1024 + 16 * lane);
        // the scales once per block, with half 0 (the loop derives half 1's
        // scale pairs from them too)
        if (half == 0) r.hd = ld16(blk + 2048 + 16 * n);
    } else if constexpr (T == LQ_Q6_K) {
        r.ql = ld16(blk + half * 1024 + 16 * lane);
        r.qh = ld16(blk + 2048 + 16 * lane);
        r.sc = ld16(blk + 3072 + 16 * n);
        r.d = *reinterpret_cast<const uint16_t *>(blk + 3328 + 2 * n);
    } else {
        r.p0 = ld16(blk + 2 * half * 1024 + 16 * lane);
        r.p1 = ld16(blk + (2 * half + 1) * 1024 + 16 * lane);
        r.dd = ld16(blk + 4096 + 16 * n);
    }
    return r;
}

// Q4_K sub-block scale pair {d * sc, dmin * mn} (packed f16, each rounded
// once) of row lane % 16, sub-block 4 HALF + lane / 16: the four lane groups
// of a wave cover the four sub-blocks of a half at once; gt_b fetches the
// pair of its own sub-block from the lane that computed it
template <int HALF>
__device__ __forceinline__ uint32_t gt_q4k_pair(const uint4 &hd, int q) {
    const uint32_t s0 = hd.y, s4 = hd.z, s8 = hd.w;   // scale bytes 0..3, 4..7, 8..11
    uint32_t sc, mn;
    if constexpr (HALF == 0) {
        sc = __builtin_amdgcn_ubfe(s0, 8 * q, 6);
        mn = __builtin_amdgcn_ubfe(s4, 8 * q, 6);
    } else {
        sc = __builtin_amdgcn_ubfe(s8, 8 * q, 4) | (__builtin_amdgcn_ubfe(s0, 8 * q + 6, 2) << 4);
        mn = __builtin_amdgcn_ubfe(s8, 8 * q + 4, 4) | (__builtin_amdgcn_ubfe(s4, 8 * q + 6, 2) << 4);
    }
    // packed f16: {sc, mn} exactly (0x6400 | n reads as 1024 + n), times
    // {d, dmin} rounds d * sc and dmin * mn once each
    const lq_h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const lq_h2 scmn = __builtin_bit_cast(lq_h2, sc | (mn << 16) | 0x64006400u) - k1024;
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(lq_h2, hd.x) * scmn);
}

// B operand (8 f16) of slice kk (0..3) of half HALF of the block, lane group
// q; Q4_K: pair = the slice's scale pair for the lane's row (gt_q4k_pair)
template <int T, int HALF, int KK>
__device__ __forceinline__ lq_h8 gt_b(const GtRaw<T> &r, int q, uint32_t pair_ab = 0) {
    uint4 o;
    if constexpr (T == LQ_Q4_K) {
        // group g = 4 HALF + KK: qs chunk g / 2 (bytes 8 ((g / 2) % 2) ..), nibble g % 2;
        // a value is round(a * q - b) from the exact q (one fused multiply-add)
        constexpr int g = 4 * HALF + KK, hb = (g >> 1) & 1, nib = g & 1;
        const lq_h2 ab = __builtin_bit_cast(lq_h2, pair_ab);
        const lq_h2 a2 = {ab.x, ab.x}, nb2 = {-ab.y, -ab.y};
        const uint32_t w0 = ((hb ? r.qs.z : r.qs.x) >> (4 * nib)) & 0x0F0F0F0Fu;
        const uint32_t w1 = ((hb ? r.qs.w : r.qs.y) >> (4 * nib)) & 0x0F0F0F0Fu;
        // the byte 0000qqqq read as FP8 e4m3 is exactly q 2^-9 (subnormal
        // below 8, normal from 8 on); the scaled conversion times 2^9 gives
        // two f16 q exactly in one instruction
        auto fma2 = [&](lq_h2 q) { return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, a2, nb2)); };
        o.x = fma2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.0f, false));
        o.y = fma2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.0f, true));
        o.z = fma2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.0f, false));
        o.w = fma2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.0f, true));
    } else if constexpr (T == LQ_Q6_K) {
        // slice g = 4 HALF + KK: values 128 HALF + 32 KK + 8q .. ; ql nibble KK / 2 of
        // bytes 8 (KK % 2) ..; qh bits 2 KK of bytes 8 HALF ..; sub-block 2g + q / 2
        constexpr int g = 4 * HALF + KK;
        const uint32_t l0 = ((KK & 1) ? r.ql.z : r.ql.x) >> (4 * (KK >> 1));
        const uint32_t l1 = ((KK & 1) ? r.ql.w : r.ql.y) >> (4 * (KK >> 1));
        const uint32_t e0 = (HALF ? r.qh.z : r.qh.x) >> (2 * KK), e1 = (HALF ? r.qh.w : r.qh.y) >> (2 * KK);
        const uint32_t w0 = (l0 & 0x0F0F0F0Fu) | ((e0 & 0x03030303u) << 4);
        const uint32_t w1 = (l1 & 0x0F0F0F0Fu) | ((e1 & 0x03030303u) << 4);
        // sub-blocks 2g and 2g + 1 share scale dword g / 2
        const uint32_t sw = (g >> 1) == 0 ? r.sc.x : (g >> 1) == 1 ? r.sc.y : (g >> 1) == 2 ? r.sc.z : r.sc.w;
        const int sbyte = ((2 * g) & 3) + (q >> 1);
        // packed f16: 1024 + q minus 1056 is q - 32 exactly; times d * sc
        // (rounded once) rounds each value once
        const _Float16 dsc = __builtin_bit_cast(_Float16, (uint16_t)(r.d & 0xFFFFu)) *
                             (_Float16)(int)__builtin_amdgcn_sbfe((int)sw, 8 * sbyte, 8);
        const lq_h2 d2 = {dsc, dsc}, k1056 = {(_Float16)1056.0f, (_Float16)1056.0f};
        auto pair = [&](uint32_t bits) {
            return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(lq_h2, bits) - k1056) * d2);
        };
        o.x = pair(f16_bytes_lo(w0));
        o.y = pair(f16_bytes_hi(w0));
        o.z = pair(f16_bytes_lo(w1));
        o.w = pair(f16_bytes_hi(w1));
    } else {
        // GGML block 4 HALF + KK: piece KK / 2 of the half, bytes 8 (KK % 2) ..
        const uint4 pc = (KK >> 1) ? r.p1 : r.p0;
        const uint32_t w0 = (KK & 1) ? pc.z : pc.x, w1 = (KK & 1) ? pc.w : pc.y;
        constexpr int g = 4 * HALF + KK;
        const uint32_t dw = g < 2 ? r.dd.x : g < 4 ? r.dd.y : g < 6 ? r.dd.z : r.dd.w;
        const uint32_t dh = (dw >> (16 * (g & 1))) & 0xFFFFu;
        const lq_h2 d2 = __builtin_bit_cast(lq_h2, dh * 0x10001u);
        q8_pairs(w0, d2, o.x, o.y);
        q8_pairs(w1, d2, o.z, o.w);
    }
    return __builtin_bit_cast(lq_h8, o);
}

// MFMAs of the four 32-value slices of half HALF of a block: B operands
// decoded from the wave's two row tiles, A operands from the LDS x tile
// x tile in LDS: [token][16 chunks of 8 halves], chunk c of token t stored at
// position c ^ (t % 16), so the 16 tokens of an A read hit 16 bank groups.
// The wave raises its priority while it issues a slice's MFMAs, so the wave
// that holds ready MFMAs keeps the matrix core of its SIMD (the waves of a
// SIMD come from different workgroups). Dense 14336 x 4096 x 512 Q8_0: 88 us
// against 97 us; the expert GEMMs gain about 1 %.
// Q4_K: pr0 / pr1 are the scale pairs of this half (gt_q4k_pair), computed
// by the caller while half 0's scale registers are live
template <int T, int HALF, int NI>
__device__ __forceinline__ void gt_half(const GtRaw<T> &w0, const GtRaw<T> &w1, const _Float16 *xs, int lane,
                                        lq_f4 (&acc)[NI][2], uint32_t pr0 = 0, uint32_t pr1 = 0) {
    const int fr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        // all A reads of the slice in flight while the B operands are decoded
        lq_h8 av[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            av[i] = *reinterpret_cast<const lq_h8 *>(xs + (16 * i + fr) * GM_BK + 8 * ((4 * kk + q) ^ fr));
        uint32_t p0 = 0, p1 = 0;
        if constexpr (T == LQ_Q4_K) {
            // the pair of sub-block 4 HALF + kk of the lane's row: lane fr + 16 kk
            const int src = 4 * (fr + 16 * kk);
            p0 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)pr0);
            p1 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)pr1);
        }
        lq_h8 b0, b1;
        if (kk == 0) { b0 = gt_b<T, HALF, 0>(w0, q, p0); b1 = gt_b<T, HALF, 0>(w1, q, p1); }
        else if (kk == 1) { b0 = gt_b<T, HALF, 1>(w0, q, p0); b1 = gt_b<T, HALF, 1>(w1, q, p1); }
        else if (kk == 2) { b0 = gt_b<T, HALF, 2>(w0, q, p0); b1 = gt_b<T, HALF, 2>(w1, q, p1); }
        else { b0 = gt_b<T, HALF, 3>(w0, q, p0); b1 = gt_b<T, HALF, 3>(w1, q, p1); }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], b0, acc[i][0], 0, 0, 0);
            acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], b1, acc[i][1], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    }
}

// Waits for the loads of gt_load<T>(.., HALF, ..) into r (the compiler places
// the wait before these empty asm statements, which read and rewrite the
// loaded registers)
__device__ __forceinline__ void gt_touch(uint4 &v) {
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    u4v t = __builtin_bit_cast(u4v, v);
    asm volatile("" : "+v"(t));
    v = __builtin_bit_cast(uint4, t);
}
template <int T, int HALF>
__device__ __forceinline__ void gt_ready(GtRaw<T> &r) {
    if constexpr (T == LQ_Q4_K) {
        gt_touch(r.qs);
        if constexpr (HALF == 0) gt_touch(r.hd);
    } else if constexpr (T == LQ_Q6_K) {
        gt_touch(r.ql);
        gt_touch(r.qh);
        gt_touch(r.sc);
        asm volatile("" : "+v"(r.d));
    } else {
        gt_touch(r.p0);
        gt_touch(r.p1);
        gt_touch(r.dd);
    }
}

// Global loads gt_load<T> issues for one row tile's half HALF
template <int T, int HALF>
constexpr int gt_loads() {
    return T == LQ_Q4_K ? (HALF == 0 ? 2 : 1) : T == LQ_Q6_K ? 4 : 3;
}

// The K loop and epilogue of one workgroup with NV 16-token MFMA tiles of
// the BN holding tokens: expert tiles end partway, and each NV is its own
// copy of the loop (no per-MFMA branches, which made the compiler copy the
// accumulators around every conditional MFMA).
template <int T, int BN, int MODE, int NW, int NV>
__device__ __forceinline__ void gt_main(const GemmArgs &a, _Float16 (*Xs)[BN * GM_BK], float *tsc, float *asc,
                                        const float *wn, const uint8_t *w0p, const uint8_t *w1p, int64_t p0, int tn,
                                        int64_t t0, int64_t t1, int64_t tiles, int64_t nsb) {
    constexpr int XN = BN * 16 / (64 * NW);   // 16-byte x chunks per thread and step
    constexpr int BB = mt_block_bytes(T);
    const lq_geom &g = a.g;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();

    // x loader: instruction i of wave w fills tile chunks (NW i + w) * 64 + lane,
    // i.e. token row (NW i + w) * 4 + lane / 16, position lane % 16, from the
    // row's chunk (lane % 16) ^ (row % 16); straight from global memory into
    // LDS (no registers), waited for with vmcnt before the step's barrier.
    // Rows of the MFMA tiles past NV are not read.
    const _Float16 *xsrc[XN];
#pragma unroll
    for (int i = 0; i < XN; ++i) {
        const int row = (NW * i + wave) * 4 + (lane >> 4), c = (lane & 15) ^ (row & 15);
        xsrc[i] = a.Xh + gemm_xrow(a, p0 + (row < tn ? row : 0)) * a.ldh + 8 * c;
    }
    // The copies are asm (cu_dma): the compiler, which sees a builtin copy as
    // an LDS write it cannot place, waited for every load (vmcnt(0)) before
    // the first LDS read after one, the weight loads just issued included.
    // Their completion before the LDS reads is the kernel's own wait before
    // each barrier.
    const uint32_t xs0 = (uint32_t)(uintptr_t)&Xs[0][0];
    auto load_x = [&](int buf, int64_t step) {
#pragma unroll
        for (int i = 0; i < XN; ++i)
            if ((NW * i + wave) * 4 < 16 * NV)   // uniform per wave
                cu_dma(xsrc[i] + step * GM_BK, xs0 + (uint32_t)(buf * BN * GM_BK * 2 + (NW * i + wave) * 64 * 16));
    };

    lq_f4 acc[NV][2];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        acc[i][0] = lq_f4{0.0f, 0.0f, 0.0f, 0.0f};
        acc[i][1] = lq_f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // prologue: half 0 of block 0, and each token's output scale (one
    // lookup per token rather than one per output value)
    GtRaw<T> a0 = gt_load<T>(w0p, 0, lane), a1 = gt_load<T>(w1p, 0, lane);
    load_x(0, 0);
    if (tid < BN) {
        const int64_t xr = gemm_xrow(a, p0 + (tid < tn ? tid : 0));
        tsc[tid] = a.inv[xr];
        if constexpr (MODE == GM_MOE_GATE_UP) {
            if (a.Yh) {
                // |silu(g) u| <= |g| |u| <= |gate row| |up row| |h|^2 (Cauchy-
                // Schwarz), times 4 for the rounding of the f16 operands, the
                // sums and the fast SiLU; 2^s brings the bound into [2^14,
                // 2^15), so no output overflows f16 (s = 0 for a zero or
                // non-finite bound, x_to_f16_row's rule)
                const double b = 4.0 * (double)wn[0] * (double)wn[1] * (double)a.xnorm2[xr];
                int s = 0;
                if (b > 0.0 && b <= 1.0e300) {
                    int e;
                    frexp(b, &e);
                    s = 15 - e;
                    s = s > 120 ? 120 : s < -120 ? -120 : s;
                }
                asc[tid] = ldexpf(1.0f, s);
                if (blockIdx.x == 0 && tid < tn) a.inv_out[p0 + tid] = ldexpf(1.0f, -s);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // step loop over blocks: half 0 from Xs[0] / (a0, a1), half 1 from Xs[1] /
    // (b0, b1). Each half waits for its own weights (requested one half
    // earlier), then requests the next half's x copy and, after it, the next
    // half's weights, so the wait before the barrier (vmcnt = those weight
    // loads) retires only the copy: the weights stay in flight across it.
    for (int64_t sb = 0; sb < nsb; ++sb) {
        gt_ready<T, 0>(a0);
        gt_ready<T, 0>(a1);
        // Q4_K: both halves' scale pairs now, so the block's scale registers
        // die in half 0 and the next block's scales load straight into them
        // (kept live into half 1, the compiler copied each freshly loaded
        // scale register and waited for the load right after issuing it)
        uint32_t p00 = 0, p01 = 0, p10 = 0, p11 = 0;
        if constexpr (T == LQ_Q4_K) {
            const int q = lane >> 4;
            p00 = gt_q4k_pair<0>(a0.hd, q);
            p01 = gt_q4k_pair<0>(a1.hd, q);
            p10 = gt_q4k_pair<1>(a0.hd, q);
            p11 = gt_q4k_pair<1>(a1.hd, q);
        }
        load_x(1, 2 * sb + 1);
        GtRaw<T> b0 = gt_load<T>(w0p + sb * BB, 1, lane), b1 = gt_load<T>(w1p + sb * BB, 1, lane);
        // nothing crosses: the loads stay ahead of the MFMAs
        __builtin_amdgcn_sched_barrier(0);
        gt_half<T, 0, NV>(a0, a1, Xs[0], lane, acc, p00, p01);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * gt_loads<T, 1>()) : "memory");
        __syncthreads();
        gt_ready<T, 1>(b0);
        gt_ready<T, 1>(b1);
        // next block (the last block re-reads itself: Xs[0] is not read again)
        const int64_t nx = sb + 1 < nsb ? sb + 1 : sb;
        load_x(0, 2 * nx);
        a0 = gt_load<T>(w0p + nx * BB, 0, lane);
        a1 = gt_load<T>(w1p + nx * BB, 0, lane);
        __builtin_amdgcn_sched_barrier(0);
        gt_half<T, 1, NV>(b0, b1, Xs[1], lane, acc, p10, p11);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * gt_loads<T, 0>()) : "memory");
        __syncthreads();
    }
    // D[m][n]: lane holds tokens 4 (lane / 16) + v of token tile i, row lane % 16 of row tile j.
    // Addresses advance from one base per row; 32-bit offsets (a tile spans
    // at most BN rows of Y)
    const int fr = lane & 15;
    if constexpr (MODE == GM_MOE_GATE_UP) {
        const int64_t r = t0 * MT_ROWS + fr;
        const bool rok = r < a.inter;
        if (a.Yh) {
            // the f16 rows the down GEMM reads: the same f32 value times
            // 2^s, rounded once (as x_to_f16_row rounds it)
            _Float16 *hb = a.Yh + p0 * a.ldy + r;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int lt = 16 * i + 4 * (lane >> 4) + v;
                    if (lt >= tn || !rok) continue;
                    const float sc = tsc[lt];
                    const float y = silu_fast(acc[i][0][v] * sc) * (acc[i][1][v] * sc);
                    hb[(uint32_t)lt * (uint32_t)a.ldy] = (_Float16)(y * asc[lt]);
                }
            }
        } else {
            float *yb = a.Y + p0 * a.y_ts + r;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int lt = 16 * i + 4 * (lane >> 4) + v;
                    if (lt >= tn || !rok) continue;
                    const float sc = tsc[lt];
                    yb[(uint32_t)lt * (uint32_t)a.y_ts] = silu_fast(acc[i][0][v] * sc) * (acc[i][1][v] * sc);
                }
            }
        }
    } else {
        const int64_t r0 = t0 * MT_ROWS + fr, r1 = t1 * MT_ROWS + fr;
        const bool ok0 = t0 < tiles && r0 < g.rows, ok1 = t1 < tiles && r1 < g.rows;
        float *yb0 = a.Y + p0 * a.y_ts + r0 * a.y_rs, *yb1 = a.Y + p0 * a.y_ts + r1 * a.y_rs;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int lt = 16 * i + 4 * (lane >> 4) + v;
                if (lt >= tn) continue;
                const float sc = tsc[lt];
                const uint32_t o = (uint32_t)lt * (uint32_t)a.y_ts;
                if (ok0) yb0[o] = acc[i][0][v] * sc;
                if (ok1) yb1[o] = acc[i][1][v] * sc;
            }
        }
    }
}

// NW waves per workgroup (4 or 8): 32 NW weight rows (gate_up: 16 NW gate and
// 16 NW up rows) share one staged x tile; 8 waves halve the x bytes each
// weight byte brings along (the MoE expert tiles)
template <int T, int BN, int MODE, int NW = 4>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gemm_tile_kernel(GemmArgs a) {
    constexpr int NI = BN / 16;            // 16-token MFMA tiles per wave
    constexpr int BB = mt_block_bytes(T);
    __shared__ __attribute__((aligned(16))) _Float16 Xs[2][BN * GM_BK];
    __shared__ float tsc[BN];              // the output scale of each token of the tile
    __shared__ float asc[MODE == GM_MOE_GATE_UP ? BN : 1];   // gate_up with f16 output: its scale per token
    const lq_geom &g = a.g;
    // wave index made wave-uniform: row-tile addresses go to scalar registers
    // (MoE Q4_K GEMMs 162 -> 128 VGPRs; gate_up 85 -> 81 us, down 55 -> 48 us)
    const int wave = wave_id();
    const uint8_t *Wt = a.Wt;
    int64_t p0;
    int tn;
    int64_t blk;
    const float *wn = nullptr;   // the expert's row norms (gate_up with f16 output)
    if constexpr (MODE == GM_DENSE) {
        // 1-D grid, padded to a multiple of 8; workgroup id -> logical index
        // xcd * per + id / 8 walks the row blocks of one token tile per XCD
        const int id = blockIdx.x, per = gridDim.x / 8;
        const int L = (id % 8) * per + id / 8;
        const int nrb = (int)((g.rows + 32 * NW - 1) / (32 * NW));
        const int64_t ntt = (a.ntok + BN - 1) / BN;
        if (L >= nrb * ntt) return;
        blk = L % nrb;
        p0 = (int64_t)(L / nrb) * BN;
        tn = (int)(a.ntok - p0 < BN ? a.ntok - p0 : BN);
    } else {
        blk = blockIdx.x;
        const int tile = blockIdx.y;
        if (tile >= a.n_tiles[0]) return;
        Wt += (int64_t)a.tile_e[tile] * a.wt_bytes;
        if (a.wnorm) wn = a.wnorm + 2 * (int64_t)a.tile_e[tile];
        p0 = a.tile_p0[tile];
        tn = a.tile_n[tile];
    }
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS, nsb = mt_nsb(g);
    // the wave's two row tiles: dense / down 2 NW blk + 2 wave + j; gate_up
    // gate tile NW blk + wave (j = 0) and its up tile inter / 16 + NW blk + wave
    int64_t t0, t1;
    if constexpr (MODE == GM_MOE_GATE_UP) {
        t0 = NW * blk + wave;
        t1 = a.inter / MT_ROWS + NW * blk + wave;
    } else {
        t0 = 2 * NW * blk + 2 * wave;
        t1 = t0 + 1;
    }
    const uint8_t *w0p = Wt + (t0 < tiles ? t0 : tiles - 1) * nsb * BB;
    const uint8_t *w1p = Wt + (t1 < tiles ? t1 : tiles - 1) * nsb * BB;
    if constexpr (MODE == GM_DENSE || NI != 4) {
        gt_main<T, BN, MODE, NW, NI>(a, Xs, tsc, asc, wn, w0p, w1p, p0, tn, t0, t1, tiles, nsb);
    } else {
        // expert tiles: one copy of the loop per count of 16-token tiles
        const int nv = __builtin_amdgcn_readfirstlane((tn + 15) >> 4);
        if (nv == 1) gt_main<T, BN, MODE, NW, 1>(a, Xs, tsc, asc, wn, w0p, w1p, p0, tn, t0, t1, tiles, nsb);
        else if (nv == 2) gt_main<T, BN, MODE, NW, 2>(a, Xs, tsc, asc, wn, w0p, w1p, p0, tn, t0, t1, tiles, nsb);
        else if (nv == 3) gt_main<T, BN, MODE, NW, 3>(a, Xs, tsc, asc, wn, w0p, w1p, p0, tn, t0, t1, tiles, nsb);
        else gt_main<T, BN, MODE, NW, 4>(a, Xs, tsc, asc, wn, w0p, w1p, p0, tn, t0, t1, tiles, nsb);
    }
}

// ---------------------------------------------------------------- CU-tile GEMM (Q8_0, many tokens)

// One workgroup per CU owns a 224-row x 128-token output tile (14 row tiles
// x 8 token tiles; 14336 x 512 is exactly 256 such tiles). The shape follows
// from what a CU can be fed: L2 delivers about 32 B per clock to a CU (1 KB
// contiguous per load instruction; half that for 64-byte pieces of rows 8 KB
// apart). Per 64-value K step the tile needs 128 tokens x 128 B of x and 224
// rows x 68 B of Q8_0 weights, about 31 KB, roughly what L2 delivers in the
// time of the step's MFMAs.
//
// Waves 0..6 compute: wave w owns row tiles 2w, 2w + 1 for all 8 token tiles
// (32 v_mfma_f32_16x16x32_f16 per step). It loads its own raw weights (tile
// form, 1 KB contiguous per load) and decodes them in registers straight into
// MFMA A operands, so weights never pass through LDS. x (the tiled form of
// x_to_f16, 16 KB per step: 8 token tiles x 2 slices, 1 KB each in lane
// order) goes into a 4-step LDS ring three steps ahead, wave w copying token
// tile w with global_load_lds; the compute waves read it as B operands (one
// conflict-free ds_read_b128 per token tile and slice). With the weights as
// A and the tokens as B, each lane ends up holding 4 consecutive rows of one
// token, stored as one 16-byte write. Ring slot (j + 3) % 4 is refilled at
// step j, after the barrier that ended step j - 1, its last reader. One
// workgroup barrier per step.
//
// The compute waves' weight loads are asm whose completion the kernel counts
// itself (4 loads per step); every use goes through cu_wait_w, which
// names the registers, and the build checks the generated code for any
// instruction touching a register whose load may still be in flight. The
// MFMAs are asm with the accumulators in VGPRs: as builtins, the register
// allocator rotated the accumulators through copies at every iteration of
// the unrolled loop, and in AGPRs the compiler capped the VGPRs at 128 and
// spilled (copied) registers with loads in flight into AGPRs.
constexpr int CU_RT = 14;                        // row tiles per workgroup
constexpr int CU_TT = 8;                         // token tiles per workgroup
constexpr int CU_WR = 2;                         // row tiles per compute wave
constexpr int CU_NC = 7;                         // compute waves
constexpr int CU_RING = 4;                       // x ring depth (steps)
constexpr int CU_XSTEP = CU_TT * 2 * 1024;       // x bytes per step
constexpr int CU_TOKENS = CU_TT * 16;
// LDS requested per workgroup: more than half of a CU's 160 KB (the ring uses
// 64 KB), so that no CU holds two workgroups (a second one would halve that
// CU's MFMA rate and leave another CU idle)
constexpr int CU_LDS_RESERVE = 96 * 1024;
static_assert(CU_RING * CU_XSTEP <= CU_LDS_RESERVE, "CU-tile LDS");

// global loads with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset (fewer VGPRs than 64-bit addresses per load)
__device__ __forceinline__ void cu_load(mt_i4 &v, const void *base, uint32_t off) {
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base) : "memory");
}
__device__ __forceinline__ void cu_load(int &v, const void *base, uint32_t off) {
    asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(off), "s"(base) : "memory");
}
template <int N, class W>
__device__ __forceinline__ void cu_wait_w(W &w) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(w[0].q), "+v"(w[0].d), "+v"(w[1].q), "+v"(w[1].d) : "n"(N) : "memory");
}

// XCD-aware tile order. Workgroups go to the 8 XCDs round robin
// (blockIdx.x % 8); renumbered, each XCD runs a contiguous range, ordered as
// groups of (up to) 4 token blocks of one row block. The 4 workgroups of a
// row block then run side by side on one XCD and read each weight step from
// its L2 (HBM reads the 62 MB of 14336 x 4096 weights once), and the XCD's
// workgroups, all at similar K positions, share the x steps in L2 as well.
__device__ __forceinline__ void cu_tile(int nrb, int ntb, int &rb, int &tb) {
    const int G = gridDim.x, per = G / 8, rem = G % 8, xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
    const int L = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int tq = L / (4 * nrb), r = L % (4 * nrb), gs = ntb - 4 * tq < 4 ? ntb - 4 * tq : 4;
    rb = r / gs;
    tb = 4 * tq + r % gs;
}

// y_vec: Y rows are contiguous (y_rs 1), 16-byte aligned, y_ts % 4 == 0
__global__ __launch_bounds__(512, 1) void gemm_cu_q80_kernel(GemmArgs a, int nrb, int ntb, int y_vec) {
    extern __shared__ __attribute__((aligned(16))) uint8_t cu_lds[];
    const lq_geom &g = a.g;
    const int lane = lane_id(), w = wave_id();
    int rb, tb;
    cu_tile(nrb, ntb, rb, tb);
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS, nsb = mt_nsb(g);
    const int64_t p0 = (int64_t)tb * CU_TOKENS, t0 = (int64_t)rb * CU_RT;
    const int nsteps = (int)(nsb * 4);               // 64-value steps (a multiple of 4)

    // x: wave w copies token tile w (both 32-value slices, 2 KB) of each step
    // into the ring; the compute waves read every token tile
    const int64_t nks = a.ldh / 32, ttiles = (a.ntok + 15) / 16;
    int64_t xtt = p0 / 16 + w;
    xtt = xtt < ttiles ? xtt : ttiles - 1;
    const uint8_t *const xsrc = reinterpret_cast<const uint8_t *>(a.Xh) + xtt * nks * 1024 + 16 * lane;
    const uint32_t ring = (uint32_t)(uintptr_t)cu_lds + 2048 * w;
    auto dma = [&](int j) {                          // 2 loads
        const int jj = j < nsteps ? j : nsteps - 1;
        const uint32_t dst = ring + (j % CU_RING) * CU_XSTEP;
        cu_dma(xsrc + 2048 * jj, dst);
        cu_dma(xsrc + 2048 * jj + 1024, dst + 1024);
    };
    dma(0);
    dma(1);
    dma(2);

    if (w == CU_NC) {
        // ---- the eighth wave only copies: x(j + 1) (requested at step j - 2)
        // is complete once at most the 4 loads of steps j - 1 and j are in flight
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int j = 0; j < nsteps; ++j) {
            dma(j + 3);
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            cu_barrier();
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---- compute waves
    uint32_t woff[CU_WR];
#pragma unroll
    for (int r = 0; r < CU_WR; ++r) {
        int64_t t = t0 + CU_WR * w + r;
        t = t < tiles ? t : tiles - 1;
        woff[r] = (uint32_t)(t * nsb * MT_Q80_BLOCK);
    }
    const uint32_t qlane = 16 * lane, dlane = 4096 + 16 * (lane & 15);
    struct WRaw { mt_i4 q; int d; };
    auto load_w = [&](WRaw (&dst)[CU_WR], int j) {    // 4 loads
        j = j < nsteps ? j : nsteps - 1;
        const int blk = j >> 2, piece = j & 3;
        const uint8_t *qb = a.Wt + (int64_t)blk * MT_Q80_BLOCK + piece * 1024, *db = a.Wt + (int64_t)blk * MT_Q80_BLOCK + 4 * piece;
#pragma unroll
        for (int r = 0; r < CU_WR; ++r) {
            cu_load(dst[r].q, qb, woff[r] + qlane);
            cu_load(dst[r].d, db, woff[r] + dlane);
        }
    };
    typedef lq_h8 WOps[CU_WR][2];
    auto decode = [&](WRaw (&src)[CU_WR], WOps &o) {
#pragma unroll
        for (int r = 0; r < CU_WR; ++r) {
            const uint32_t d = (uint32_t)src[r].d;
            const lq_h2 d0 = __builtin_bit_cast(lq_h2, (d & 0xFFFFu) * 0x10001u);
            const lq_h2 d1 = __builtin_bit_cast(lq_h2, (d >> 16) * 0x10001u);
            uint4 o0, o1;
            q8_pairs((uint32_t)src[r].q[0], d0, o0.x, o0.y);
            q8_pairs((uint32_t)src[r].q[1], d0, o0.z, o0.w);
            q8_pairs((uint32_t)src[r].q[2], d1, o1.x, o1.y);
            q8_pairs((uint32_t)src[r].q[3], d1, o1.z, o1.w);
            o[r][0] = __builtin_bit_cast(lq_h8, o0);
            o[r][1] = __builtin_bit_cast(lq_h8, o1);
        }
    };

    lq_f4 acc[CU_WR][CU_TT];
#pragma unroll
    for (int r = 0; r < CU_WR; ++r)
#pragma unroll
        for (int i = 0; i < CU_TT; ++i) acc[r][i] = lq_f4{0.0f, 0.0f, 0.0f, 0.0f};

    // x B operands: slice sl of step j is read into xv[sl] as soon as the
    // MFMAs of slice sl of step j - 1 are issued (x(j) has been in LDS since
    // the barrier that ended step j - 2), so the reads overlap MFMAs
    typedef lq_h8 XOps[2][CU_TT];
    auto read_x = [&](int j, XOps &xv, int sl) {
        const uint8_t *xs = cu_lds + (j % CU_RING) * CU_XSTEP + 16 * lane + sl * 1024;
#pragma unroll
        for (int i = 0; i < CU_TT; ++i) xv[sl][i] = *reinterpret_cast<const lq_h8 *>(xs + 2048 * i);
    };
    auto mfmas = [&](int j, XOps &xv, WOps &cur) {
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
            for (int i = 0; i < CU_TT; ++i)
#pragma unroll
                for (int r = 0; r < CU_WR; ++r)
                    asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc[r][i]) : "v"(cur[r][sl]), "v"(xv[sl][i]));
            read_x(j + 1, xv, sl);
        }
    };

    // Raw weights run 4 steps ahead in 4 register sets. Each step a compute
    // wave requests its 2 KB of x(j + 3), then 4 weight loads: the raw set
    // decoded at step j was requested at step j - 4 and is complete once at
    // most the 18 loads of steps j - 3 .. j - 1 are in flight; the wave's own
    // part of x(j + 1), requested at step j - 2, once at most 16 are (the
    // weights of step j - 2 and steps j - 1, j), and the barrier then makes
    // all of x(j + 1) visible. One decoded operand set: the MFMAs read their
    // operands at issue, so the decode may overwrite them once the step's
    // MFMAs are issued. The two compute waves of a SIMD (w and w + 4) run
    // opposite phases, one issuing MFMAs while the other decodes:
    //   waves 0..3, step j: MFMAs(j); decode W(j + 1); request x(j + 3), W(j + 5)
    //   waves 4..6, step j: decode W(j); request x(j + 3), W(j + 4); MFMAs(j)
    // Everything the prologue requested has landed before the loop: the
    // compiler may copy loop-carried registers on entry, and a copy of a
    // register still waiting for its load would read stale data.
    WRaw wr[4][CU_WR];
    WOps cur;
    XOps xv;
    if (w < 4) {
        WRaw w0[CU_WR];
        load_w(w0, 0);
#pragma unroll
        for (int k = 1; k <= 4; ++k) load_w(wr[k & 3], k);
        cu_wait_w<16>(w0);
        decode(w0, cur);
#pragma unroll
        for (int k = 0; k < 4; ++k) cu_wait_w<0>(wr[k]);
        __syncthreads();
        read_x(0, xv, 0);
        read_x(0, xv, 1);
        auto step = [&](int j, WRaw (&w1)[CU_WR]) {
            mfmas(j, xv, cur);
            cu_wait_w<18>(w1);
            decode(w1, cur);                    // past the end: a clamped copy nobody uses
            dma(j + 3);
            load_w(w1, j + 5);
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");   // own part of x(j + 1)
            cu_barrier();
        };
        for (int j = 0; j < nsteps; j += 4) {
            step(j, wr[1]);
            step(j + 1, wr[2]);
            step(j + 2, wr[3]);
            step(j + 3, wr[0]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) load_w(wr[k], k);
#pragma unroll
        for (int k = 0; k < 4; ++k) cu_wait_w<0>(wr[k]);
        __syncthreads();
        read_x(0, xv, 0);
        read_x(0, xv, 1);
        auto step = [&](int j, WRaw (&w0)[CU_WR]) {
            cu_wait_w<18>(w0);
            decode(w0, cur);
            dma(j + 3);
            load_w(w0, j + 4);
            mfmas(j, xv, cur);
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");   // own part of x(j + 1)
            cu_barrier();
        };
        for (int j = 0; j < nsteps; j += 4) {
            step(j, wr[0]);
            step(j + 1, wr[1]);
            step(j + 2, wr[2]);
            step(j + 3, wr[3]);
        }
    }
    // the loads past the end land in registers the compiler counts as free;
    // and the MFMAs are asm, so the compiler does not know to wait for their
    // results before reading the accumulators: 24 wait states cover the
    // longest (16-pass) MFMA write-to-read distance
    asm volatile("s_waitcnt vmcnt(0)\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");

    // D: lane holds rows 4 (lane / 16) + v of a row tile, token lane % 16 of a token tile
#pragma unroll
    for (int i = 0; i < CU_TT; ++i) {
        const int64_t p = p0 + 16 * i + (lane & 15);
        if (p >= a.ntok) continue;
        const float sc = a.inv[p];
        float *yp = a.Y + p * a.y_ts;
#pragma unroll
        for (int r = 0; r < CU_WR; ++r) {
            const int64_t t = t0 + CU_WR * w + r, row = t * MT_ROWS + 4 * (lane >> 4);
            if (t >= tiles) continue;
            const lq_f4 v = acc[r][i] * sc;
            if (y_vec && row + 3 < g.rows) {
                *reinterpret_cast<lq_f4 *>(yp + row) = v;
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (row + k < g.rows) yp[(row + k) * a.y_rs] = v[k];
            }
        }
    }
}

// ---------------------------------------------------------------- host side

// f16 activation rows are padded with zeros to a multiple of 256 values (the
// tile form's block; a multiple of the row-plane kernel's 128-value step)
static int64_t gemm_ldh(const lq_geom &g) { return 256 * ((g.cols + 255) / 256); }

int64_t gemm_workspace_bytes(const lq_geom &g, int64_t ntok) {
    // room for the tiled form too: tokens padded to a multiple of 16
    const int64_t xh = (((ntok + 15) / 16 * 16) * gemm_ldh(g) * 2 + 255) & ~(int64_t)255;
    return xh + ntok * 4;
}

// The tiled layout with whole-line stores: workgroup b converts tokens
// 8 b .. 8 b + 7, one wave each, with the same per-row scale as
// x_to_f16_kernel, and writes them through LDS 64 value groups at a time. In
// the 1 KB slice of a 16-token group, the eight tokens' slots of one value
// octet are 128 contiguous bytes, so every store of the workgroup fills whole
// 128-byte lines (the one-wave kernel's scattered 16-byte stores wrote twice
// the bytes). Workgroup (b, y) stores chunks i = y, y + gridDim.y, ... Rows
// of at most 64 NG groups (NG <= 8); tokens ntok .. of the last 16-token
// group are written as zeros.
template <int NG>
__global__ __launch_bounds__(512) void x_to_f16_tiles_kernel(const float *__restrict__ X, int64_t ldx, int cols,
                                                             const int32_t *__restrict__ rows_map, int k,
                                                             int64_t ntok, _Float16 *__restrict__ Xh, int ldh,
                                                             float *__restrict__ inv, int vec) {
    __shared__ uint4 stage[64 * 8];   // [lane = 4 quad + octet][token, swizzled]
    const int lane = lane_id(), tw = wave_id();
    const int64_t t0 = (int64_t)blockIdx.x * 8, t = t0 + tw;
    const bool real = t < ntok;
    const int64_t src = real ? (rows_map ? (int64_t)(rows_map[t] / k) : t) : 0;
    const float *x = X + src * ldx;
    const int ngx = cols >> 3, nq = ldh >> 5;
    lq_f4 lo[NG], hi[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int gi = lane + 64 * i;
        lo[i] = hi[i] = lq_f4{0.f, 0.f, 0.f, 0.f};
        if (real && gi < ngx) {
            if (vec) {
                lo[i] = *reinterpret_cast<const lq_f4 *>(x + 8 * gi);
                hi[i] = *reinterpret_cast<const lq_f4 *>(x + 8 * gi + 4);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    lo[i][c] = x[8 * gi + c];
                    hi[i][c] = x[8 * gi + 4 + c];
                }
            }
        }
    }
    // the largest magnitude as ordered bits; NaN counts as zero (fmaxf's rule)
    uint32_t mb = 0;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float a = lo[i][c], b = hi[i][c];
            const uint32_t ua = __builtin_bit_cast(uint32_t, a) & 0x7fffffffu;
            const uint32_t ub = __builtin_bit_cast(uint32_t, b) & 0x7fffffffu;
            mb = max(mb, max(ua > 0x7f800000u ? 0u : ua, ub > 0x7f800000u ? 0u : ub));
        }
    const float m = __builtin_bit_cast(float, wave_max_u32(mb));
    int s = 0;
    if (m > 0.0f && m <= 3.4e38f) {
        int e;
        frexpf(m, &e);          // m < 2^e <= 2m
        s = 15 - e;             // m * 2^s in [2^14, 2^15)
        s = s > 120 ? 120 : s < -120 ? -120 : s;
    }
    const float sc = ldexpf(1.0f, s);
    const int64_t blk0 = (t0 >> 4) * nq;         // 1 KB slice of quad 0 of this 16-token group
    const int half = (int)((t0 >> 3) & 1);       // tokens 8 half .. 8 half + 7 of the group
    const int j = threadIdx.x, L = j >> 3, tk = j & 7;   // store: lane L's slot of token tk
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        if (i % (int)gridDim.y != (int)blockIdx.y) continue;   // this workgroup's share of the chunks
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            o[c] = (_Float16)(lo[i][c] * sc);
            o[4 + c] = (_Float16)(hi[i][c] * sc);
        }
        stage[lane * 8 + (tw ^ (lane & 7))] = __builtin_bit_cast(uint4, o);
        __syncthreads();
        const int q = 16 * i + (L >> 2);          // quad (32-value slice) of lane L's group
        if (q < nq) {
            const int64_t slot = ((blk0 + q) << 6) + 8 * half + tk + 16 * (L & 3);
            *reinterpret_cast<uint4 *>(Xh + 8 * slot) = stage[L * 8 + (tk ^ (L & 7))];
        }
        __syncthreads();
    }
    if (real && lane == 0) inv[t] = ldexpf(1.0f, -s);
}

int launch_x_to_f16(const float *X, int64_t ldx, int64_t cols, const int32_t *rows_map, int k, int64_t ntok,
                    _Float16 *Xh, int64_t ldh, float *inv, hipStream_t s, int tiled, float *nrm2) {
    if (ntok <= 0) return LOCALAI_OK;
    if (tiled && nrm2) return fail(LOCALAI_EARG, "f16 tiles: no row norms");
    if (cols % 8 || ldh % 8 || ldh < cols) return fail(LOCALAI_EARG, "f16 rows: cols % 8 != 0");
    if (tiled && ldh % 32) return fail(LOCALAI_EARG, "f16 tiles: row length % 32 != 0");
    const int vec = (uintptr_t)X % 16 == 0 && ldx % 4 == 0;
    const int per = (int)((ldh / 8 + 63) / 64);   // 8-value groups per lane
    const int64_t npad = tiled ? (ntok + 15) / 16 * 16 : ntok;
    if (tiled && per <= 8) {
        // the chunks of an 8-token group split over up to 4 workgroups (each
        // reads the whole rows for their maxima, mostly from L2), so that
        // 512 tokens occupy 256 workgroups
        const dim3 g8((unsigned)(npad / 8), (unsigned)(per < 4 ? per : 4));
        auto gt = [&](auto kern) {
            hipLaunchKernelGGL(kern, g8, dim3(512), 0, s, X, ldx, (int)cols, rows_map, k, ntok, Xh, (int)ldh, inv, vec);
        };
        if (per <= 1) gt(x_to_f16_tiles_kernel<1>);
        else if (per <= 2) gt(x_to_f16_tiles_kernel<2>);
        else if (per <= 4) gt(x_to_f16_tiles_kernel<4>);
        else gt(x_to_f16_tiles_kernel<8>);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
    // one token per wave; one-wave workgroups below 1024 tokens, so that 512
    // tokens reach every CU (four-wave workgroups left half of them idle)
    const int wpg = npad < 1024 ? 1 : 4;
    const dim3 grid((unsigned)((npad + wpg - 1) / wpg));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(64 * wpg), 0, s, X, ldx, (int)cols, rows_map, k, ntok, Xh, (int)ldh, inv,
                           vec, tiled, npad, nrm2);
    };
    if (per <= 1)
        go(x_to_f16_kernel<1>);
    else if (per <= 2)
        go(x_to_f16_kernel<2>);
    else if (per <= 4)
        go(x_to_f16_kernel<4>);
    else if (per <= 8)
        go(x_to_f16_kernel<8>);
    else
        go(x_to_f16_kernel<0>);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

template <int MODE, int BN>
static int launch_gemm_t(const GemmArgs &a, dim3 grid, hipStream_t s) {
    switch (a.g.type) {
#define LQ_GM(TT) case TT: hipLaunchKernelGGL((gemm_kernel<TT, BN, MODE>), grid, dim3(256), 0, s, a); break;
        LQ_GM(LQ_Q4_K) LQ_GM(LQ_Q5_K) LQ_GM(LQ_Q6_K) LQ_GM(LQ_Q8_0) LQ_GM(LQ_Q4_0)
#undef LQ_GM
        default: return fail(LOCALAI_ETYPE, "matmul: unsupported GGML type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

template <int MODE, int BN, int NW = 4>
static int launch_gemm_tile_t(const GemmArgs &a, dim3 grid, hipStream_t s) {
    switch (a.g.type) {
#define LQ_GT(TT) case TT: hipLaunchKernelGGL((gemm_tile_kernel<TT, BN, MODE, NW>), grid, dim3(64 * NW), 0, s, a); break;
        LQ_GT(LQ_Q4_K) LQ_GT(LQ_Q6_K) LQ_GT(LQ_Q8_0)
#undef LQ_GT
        default: return fail(LOCALAI_ETYPE, "matmul: no tile form for this GGML type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_gemm(const lq_geom &g, const uint8_t *W, const uint8_t *Wt, const float *X, int64_t ntok, float *Y,
                int64_t y_ts, int64_t y_rs, void *ws, int64_t ws_bytes, hipStream_t s) {
    if (ntok <= 0) return LOCALAI_OK;
    if (ws_bytes < gemm_workspace_bytes(g, ntok)) return fail(LOCALAI_EARG, "matmul: workspace too small");
    const int64_t ldh = gemm_ldh(g);
    _Float16 *Xh = (_Float16 *)ws;
    float *inv = (float *)((uint8_t *)ws + ((((ntok + 15) / 16 * 16) * ldh * 2 + 255) & ~(int64_t)255));
    GemmArgs a{};
    a.g = g; a.W = W; a.Xh = Xh; a.ldh = (int)ldh; a.inv = inv; a.ntok = ntok; a.Y = Y; a.y_ts = y_ts; a.y_rs = y_rs;
    a.Wt = Wt;
    // the CU-tile kernel: Q8_0 tile form, enough tokens to fill the CUs, and
    // 32-bit byte offsets into the weights and the tiled x
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    if (Wt && g.type == LQ_Q8_0 && ntok >= 256 && (size_t)CU_LDS_RESERVE <= max_lds_per_block() &&
        tiles * mt_nsb(g) * MT_Q80_BLOCK < ((int64_t)1 << 32) && (ntok + 15) / 16 * 16 * ldh * 2 < ((int64_t)1 << 32)) {
        if (int st = launch_x_to_f16(X, g.cols, g.cols, nullptr, 1, ntok, Xh, ldh, inv, s, 1)) return st;
        const int64_t nrb = (tiles + CU_RT - 1) / CU_RT, ntb = (ntok + CU_TOKENS - 1) / CU_TOKENS;
        if (nrb * ntb > ((int64_t)1 << 30)) return fail(LOCALAI_EARG, "matmul: problem too large");
        const int y_vec = y_rs == 1 && y_ts % 4 == 0 && (uintptr_t)Y % 16 == 0;
        hipLaunchKernelGGL(gemm_cu_q80_kernel, dim3((unsigned)(nrb * ntb)), dim3(512), CU_LDS_RESERVE, s, a, (int)nrb,
                           (int)ntb, y_vec);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
    if (int st = launch_x_to_f16(X, g.cols, g.cols, nullptr, 1, ntok, Xh, ldh, inv, s)) return st;
    if (Wt) {
        const int64_t nwg = ((g.rows + GT_WROWS - 1) / GT_WROWS) * ((ntok + GM_BN - 1) / GM_BN);
        if (nwg > ((int64_t)1 << 30)) return fail(LOCALAI_EARG, "matmul: problem too large");
        return launch_gemm_tile_t<GM_DENSE, GM_BN>(a, dim3((unsigned)((nwg + 7) / 8 * 8)), s);
    }
    const int64_t nwg = ((g.rows + GM_BM - 1) / GM_BM) * ((ntok + GM_BN - 1) / GM_BN);
    if (nwg > ((int64_t)1 << 30)) return fail(LOCALAI_EARG, "matmul: problem too large");
    dim3 grid((unsigned)((nwg + 7) / 8 * 8));
    return launch_gemm_t<GM_DENSE, GM_BN>(a, grid, s);
}

int moe_gemm_tile() { return GM_MOE_BN; }

int launch_moe_gemm(const lq_geom &g, const uint8_t *Wall, const uint8_t *Wt_all, int64_t wt_bytes, bool gate_up,
                    const _Float16 *Xh, int64_t ldh, const float *inv, const int32_t *rows_map, int rows_k,
                    float *Y, int64_t y_ts, int64_t inter, const int32_t *tile_e, const int32_t *tile_p0,
                    const int32_t *tile_n, const int32_t *n_tiles, int max_tiles, hipStream_t s,
                    const MoeF16Out *f16_out) {
    GemmArgs a{};
    a.g = g; a.W = Wall; a.Xh = Xh; a.ldh = (int)ldh; a.inv = inv; a.Y = Y; a.y_ts = y_ts; a.y_rs = 1;
    a.rows_map = rows_map; a.rows_k = rows_k;
    a.tile_e = tile_e; a.tile_p0 = tile_p0; a.tile_n = tile_n; a.n_tiles = n_tiles; a.inter = inter;
    a.Wt = Wt_all; a.wt_bytes = wt_bytes;
    if (max_tiles <= 0) return LOCALAI_OK;
    if (max_tiles > 65535) return fail(LOCALAI_EARG, "moe: too many token tiles");
    if (f16_out) {
        if (!gate_up || !Wt_all || inter % MT_ROWS || !f16_out->wnorm || !f16_out->xnorm2)
            return fail(LOCALAI_EARG, "moe: f16 gate_up output needs the tile form, inter % 16 == 0 and the norms");
        a.Yh = f16_out->Yh; a.ldy = f16_out->ldy; a.inv_out = f16_out->inv_out;
        a.wnorm = f16_out->wnorm; a.xnorm2 = f16_out->xnorm2;
    }
    if (Wt_all && (!gate_up || inter % MT_ROWS == 0)) {
        constexpr int NW = GM_MOE_NW;
        if (gate_up)
            return launch_gemm_tile_t<GM_MOE_GATE_UP, GM_MOE_BN, NW>(
                a, dim3((unsigned)((inter + 16 * NW - 1) / (16 * NW)), (unsigned)max_tiles), s);
        return launch_gemm_tile_t<GM_MOE_DOWN, GM_MOE_BN, NW>(
            a, dim3((unsigned)((g.rows + 32 * NW - 1) / (32 * NW)), (unsigned)max_tiles), s);
    }
    if (gate_up) {
        dim3 grid((unsigned)((inter + GM_BM / 2 - 1) / (GM_BM / 2)), (unsigned)max_tiles);
        return launch_gemm_t<GM_MOE_GATE_UP, GM_MOE_BN>(a, grid, s);
    }
    dim3 grid((unsigned)((g.rows + GM_BM - 1) / GM_BM), (unsigned)max_tiles);
    return launch_gemm_t<GM_MOE_DOWN, GM_MOE_BN>(a, grid, s);
}

}  // namespace lq
