// Prefill matmul on MFMA: Y[t, r] = sum_c W[r, c] * X[t, c] for many tokens.
//
// Counterpart of decoded_matmul_row / localai_*_matmul
// (engine/native_quant.cpp:444-531, :744-768): the reference decodes each row
// exactly to fp32 and runs fp32 FMAs over the tokens. Here a workgroup owns a
// 128-row x 128-token output tile; per 128-value K step it decodes its 128
// weight rows exactly in fp32 (the same per-type formulas as the dequant
// kernels), rounds them once to f16 into an LDS tile, stages the matching f16
// activations next to it, and 4 waves (64 x 64 outputs each) run
// v_mfma_f32_16x16x32_f16 with fp32 accumulation.
//
// Activations are converted once per call: each token row is scaled by a
// power of two so that its largest magnitude lies in [2^14, 2^15) (exact),
// rounded to f16, and the output is scaled back by the inverse power. f16 (11
// significant bits) rather than bf16 (8) keeps the normwise error near 2^-12.
#include "gemv_core.h"
#include "internal.h"

namespace lq {

typedef _Float16 lq_h8 __attribute__((ext_vector_type(8)));
typedef float lq_f4 __attribute__((ext_vector_type(4)));

constexpr int GM_BM = 128;             // weight rows per workgroup
constexpr int GM_BN = 128;             // tokens per workgroup (dense)
constexpr int GM_MOE_BN = 64;          // tokens per workgroup (MoE expert tiles)
constexpr int GM_BK = 128;             // K values per step (two 64-value units)
constexpr int GM_LD = GM_BK + 8;       // LDS row stride in halves (272 B: 16 lanes of a
                                       // 16-byte read hit 16 distinct bank groups)

// ---------------------------------------------------------------- activations

// One workgroup per token row. src row = rows_map ? rows_map[t] / k : t.
// Xh[t, 0..ldh) = f16(X[src, c] * 2^s) (zero past cols); inv[t] = 2^-s.
__global__ __launch_bounds__(256) void x_to_f16_kernel(const float *__restrict__ X, int64_t ldx, int cols,
                                                       const int32_t *__restrict__ rows_map, int k,
                                                       _Float16 *__restrict__ Xh, int ldh,
                                                       float *__restrict__ inv) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const int64_t src = rows_map ? (int64_t)(rows_map[t] / k) : (int64_t)t;
    const float *x = X + src * ldx;
    float m = 0.0f;
    for (int c = tid; c < cols; c += 256) m = fmaxf(m, fabsf(x[c]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int s = 0;
    if (m > 0.0f && m <= 3.4e38f) {
        int e;
        frexpf(m, &e);          // m < 2^e <= 2m
        s = 15 - e;             // m * 2^s in [2^14, 2^15)
        s = s > 120 ? 120 : s < -120 ? -120 : s;
    }
    _Float16 *xh = Xh + (int64_t)t * ldh;
    for (int c = tid; c < ldh; c += 256) xh[c] = (_Float16)(c < cols ? ldexpf(x[c], s) : 0.0f);
    if (tid == 0) inv[t] = ldexpf(1.0f, -s);
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

// Q8_0 weights straight to f16 pairs: byte q + 128 under the f16 exponent of
// 1024 reads as 1152 + q (exact), minus 1152 gives q exactly, and one f16
// multiply by d rounds d * q once (the same value as rounding the exact fp32
// product). Four int8 quants in `w` -> two f16 pairs.
__device__ __forceinline__ void q8_pairs(uint32_t w, lq_h2 d2, uint32_t &lo, uint32_t &hi) {
    const uint32_t b = w ^ 0x80808080u;
    const uint32_t l = (b & 0xFFu) | ((b & 0xFF00u) << 8) | 0x64006400u;
    const uint32_t h = ((b >> 16) & 0xFFu) | ((b >> 8) & 0xFF0000u) | 0x64006400u;
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
};

template <int T, int BN, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    constexpr int NI = BN / 32;            // 16-token MFMA tiles per wave (waves split tokens in 2)
    __shared__ __attribute__((aligned(16))) _Float16 Ws[GM_BM * GM_LD];
    __shared__ __attribute__((aligned(16))) _Float16 Xs[BN * GM_LD];
    const lq_geom &g = a.g;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    const int64_t xrow = p0 + (xr < tn ? xr : 0);
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
            const float sc = a.inv[p];
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

// ---------------------------------------------------------------- host side

static int64_t gemm_ldh(const lq_geom &g) { return (int64_t)GM_BK * ((g.nu + 1) / 2); }

int64_t gemm_workspace_bytes(const lq_geom &g, int64_t ntok) {
    const int64_t xh = (ntok * gemm_ldh(g) * 2 + 255) & ~(int64_t)255;
    return xh + ntok * 4;
}

int launch_x_to_f16(const float *X, int64_t ldx, int64_t cols, const int32_t *rows_map, int k, int64_t ntok,
                    _Float16 *Xh, int64_t ldh, float *inv, hipStream_t s) {
    if (ntok <= 0) return LOCALAI_OK;
    hipLaunchKernelGGL(x_to_f16_kernel, dim3((unsigned)ntok), dim3(256), 0, s, X, ldx, (int)cols, rows_map, k, Xh,
                       (int)ldh, inv);
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

int launch_gemm(const lq_geom &g, const uint8_t *W, const float *X, int64_t ntok, float *Y, int64_t y_ts,
                int64_t y_rs, void *ws, int64_t ws_bytes, hipStream_t s) {
    if (ntok <= 0) return LOCALAI_OK;
    if (ws_bytes < gemm_workspace_bytes(g, ntok)) return fail(LOCALAI_EARG, "matmul: workspace too small");
    const int64_t ldh = gemm_ldh(g);
    _Float16 *Xh = (_Float16 *)ws;
    float *inv = (float *)((uint8_t *)ws + ((ntok * ldh * 2 + 255) & ~(int64_t)255));
    if (int st = launch_x_to_f16(X, g.cols, g.cols, nullptr, 1, ntok, Xh, ldh, inv, s)) return st;
    GemmArgs a{};
    a.g = g; a.W = W; a.Xh = Xh; a.ldh = (int)ldh; a.inv = inv; a.ntok = ntok; a.Y = Y; a.y_ts = y_ts; a.y_rs = y_rs;
    const int64_t nwg = ((g.rows + GM_BM - 1) / GM_BM) * ((ntok + GM_BN - 1) / GM_BN);
    if (nwg > ((int64_t)1 << 30)) return fail(LOCALAI_EARG, "matmul: problem too large");
    dim3 grid((unsigned)((nwg + 7) / 8 * 8));
    return launch_gemm_t<GM_DENSE, GM_BN>(a, grid, s);
}

int moe_gemm_tile() { return GM_MOE_BN; }

int launch_moe_gemm(const lq_geom &g, const uint8_t *Wall, bool gate_up, const _Float16 *Xh, int64_t ldh,
                    const float *inv, float *Y, int64_t y_ts, int64_t inter, const int32_t *tile_e,
                    const int32_t *tile_p0, const int32_t *tile_n, const int32_t *n_tiles, int max_tiles,
                    hipStream_t s) {
    GemmArgs a{};
    a.g = g; a.W = Wall; a.Xh = Xh; a.ldh = (int)ldh; a.inv = inv; a.Y = Y; a.y_ts = y_ts; a.y_rs = 1;
    a.tile_e = tile_e; a.tile_p0 = tile_p0; a.tile_n = tile_n; a.n_tiles = n_tiles; a.inter = inter;
    if (max_tiles <= 0) return LOCALAI_OK;
    if (max_tiles > 65535) return fail(LOCALAI_EARG, "moe: too many token tiles");
    if (gate_up) {
        dim3 grid((unsigned)((inter + GM_BM / 2 - 1) / (GM_BM / 2)), (unsigned)max_tiles);
        return launch_gemm_t<GM_MOE_GATE_UP, GM_MOE_BN>(a, grid, s);
    }
    dim3 grid((unsigned)((g.rows + GM_BM - 1) / GM_BM), (unsigned)max_tiles);
    return launch_gemm_t<GM_MOE_DOWN, GM_MOE_BN>(a, grid, s);
}

}  // namespace lq
