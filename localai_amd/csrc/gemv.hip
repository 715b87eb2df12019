// Decode matvec over lane-interleaved weights (layout: qformat.h).
//
//   y[t, r] = sum_c W[r, c] * x[t, c],  t < NT (1..8 activation vectors)
//
// Mapping: a workgroup owns one 64-row tile; lane = row. The K dimension is
// cut into contiguous block ranges, one per wave ("bpw" blocks per wave), and
// the per-wave partial sums are added in LDS in a fixed order, so results are
// deterministic. Every weight fetch is a 16 B/lane load of one chunk for 64
// rows: 1 KiB contiguous per wave instruction. x is wave-uniform (every lane
// walks the same K position) and is read with scalar loads into SGPRs, so it
// costs no VGPRs and no LDS bandwidth.
//
// Arithmetic is fp32 on exactly decoded integer quants, following the
// factorisation of engine/native_quant.cpp:183-337 but without quantising x:
//   Q4_K/Q5_K: sum_g (d*sc_g) * sum_j q_j x_j  -  (dmin*mn_g) * sum_g(x)
//   Q6_K     : sum_s (d*sc_s) * (sum_j q6_j x_j - 32 * sum_s(x))      (16-value s)
//   Q8_0     : d * (sum_j (q_j + 128) x_j - 128 * sum_b(x))
//   Q4_0     : d * (sum_j q4_j x_j - 8 * sum_b(x))
// The group sums of x are computed once per wave by the 64 lanes together
// and broadcast through SGPRs.
#include "dev_common.h"
#include "internal.h"

namespace lq {

template <int T> struct Fmt;
template <> struct Fmt<LQ_Q4_K> { static constexpr int BV = 256, NC = 9, SG = 32; };
template <> struct Fmt<LQ_Q5_K> { static constexpr int BV = 256, NC = 11, SG = 32; };
template <> struct Fmt<LQ_Q6_K> { static constexpr int BV = 256, NC = 13, SG = 16; };
template <> struct Fmt<LQ_Q8_0> { static constexpr int BV = 32, NC = 2, SG = 32; };
template <> struct Fmt<LQ_Q4_0> { static constexpr int BV = 32, NC = 1, SG = 32; };

// x-group sums for one 256-value span starting at xs (wave-cooperative):
// lane l adds x[4l..4l+3]; groups of SG values = SG/4 lanes.
template <int SG>
__device__ __forceinline__ float span_group_sum(const float *__restrict__ xs) {
    const float4 v = reinterpret_cast<const float4 *>(xs)[lane_id()];
    float s = (v.x + v.y) + (v.z + v.w);
    return group_sum<SG / 4>(s);
}

// Dot of the 16 values of one chunk (4 dwords of packed bytes, each byte an
// unsigned quant) with 16 consecutive x values.
__device__ __forceinline__ float dot16_u8(uint4 q, const float *__restrict__ x, float acc) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t w = u4_get(q, d);
        acc = __builtin_fmaf(ubyte0(w), x[4 * d + 0], acc);
        acc = __builtin_fmaf(ubyte1(w), x[4 * d + 1], acc);
        acc = __builtin_fmaf(ubyte2(w), x[4 * d + 2], acc);
        acc = __builtin_fmaf(ubyte3(w), x[4 * d + 3], acc);
    }
    return acc;
}

__device__ __forceinline__ uint4 u4_and(uint4 a, uint32_t m) { return make_uint4(a.x & m, a.y & m, a.z & m, a.w & m); }
__device__ __forceinline__ uint4 u4_shr(uint4 a, int s) { return make_uint4(a.x >> s, a.y >> s, a.z >> s, a.w >> s); }
__device__ __forceinline__ uint4 u4_shl(uint4 a, int s) { return make_uint4(a.x << s, a.y << s, a.z << s, a.w << s); }
__device__ __forceinline__ uint4 u4_or(uint4 a, uint4 b) { return make_uint4(a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w); }

// Contribution of one block (all its values) of this lane's row to NT outputs.
// `c` holds the block's NC chunks, `d16` the block's fp16 scale if any,
// `xs[t]` points at the block's x values for vector t, `S[t][k]` are the x
// group sums (uniform).
template <int T, int NT>
__device__ __forceinline__ void block_dot(const uint4 *c, uint32_t d16, const float *const *xs,
                                          const float (*S)[16], float *acc) {
    const uint32_t M0F = opaque(0x0F0F0F0Fu), MF0 = opaque(0xF0F0F0F0u);
    const uint32_t M30 = opaque(0x30303030u);
    if constexpr (T == LQ_Q4_K || T == LQ_Q5_K) {
        const uint4 h = c[0];
        const float d = f16_to_f32(h.x), dmin = f16_to_f32(h.x >> 16);
        const uint32_t sc_lo = h.y & 0x3F3F3F3Fu;
        const uint32_t mn_lo = h.z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        float scale[8], minimum[8];
        scale[0] = d * ubyte0(sc_lo); scale[1] = d * ubyte1(sc_lo);
        scale[2] = d * ubyte2(sc_lo); scale[3] = d * ubyte3(sc_lo);
        scale[4] = d * ubyte0(sc_hi); scale[5] = d * ubyte1(sc_hi);
        scale[6] = d * ubyte2(sc_hi); scale[7] = d * ubyte3(sc_hi);
        minimum[0] = dmin * ubyte0(mn_lo); minimum[1] = dmin * ubyte1(mn_lo);
        minimum[2] = dmin * ubyte2(mn_lo); minimum[3] = dmin * ubyte3(mn_lo);
        minimum[4] = dmin * ubyte0(mn_hi); minimum[5] = dmin * ubyte1(mn_hi);
        minimum[6] = dmin * ubyte2(mn_hi); minimum[7] = dmin * ubyte3(mn_hi);
        constexpr int QS = T == LQ_Q4_K ? 1 : 3;   // first qs chunk
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            uint4 qa = c[QS + 2 * p], qb = c[QS + 2 * p + 1];
            uint4 la, lb, ha, hb;
            if constexpr (T == LQ_Q4_K) {
                // high nibbles kept in place: bytes hold 16*q, the 1/16 goes into the scale
                la = u4_and(qa, M0F); lb = u4_and(qb, M0F);
                ha = u4_and(qa, MF0); hb = u4_and(qb, MF0);
            } else {
                // 5th bit of group g is bit g of qh[j]; qh is chunks 1 (j<16) and 2 (j>=16)
                const uint4 qha = c[1], qhb = c[2];
                const int g0 = 2 * p, g1 = 2 * p + 1;
                la = u4_or(u4_and(qa, M0F), u4_shl(u4_and(u4_shr(qha, g0), 0x01010101u), 4));
                lb = u4_or(u4_and(qb, M0F), u4_shl(u4_and(u4_shr(qhb, g0), 0x01010101u), 4));
                ha = u4_or(u4_and(u4_shr(qa, 4), 0x0F0F0F0Fu), u4_shl(u4_and(u4_shr(qha, g1), 0x01010101u), 4));
                hb = u4_or(u4_and(u4_shr(qb, 4), 0x0F0F0F0Fu), u4_shl(u4_and(u4_shr(qhb, g1), 0x01010101u), 4));
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float *x = xs[t] + 64 * p;
                float s_lo = dot16_u8(la, x, 0.0f);
                s_lo = dot16_u8(lb, x + 16, s_lo);
                float s_hi = dot16_u8(ha, x + 32, 0.0f);
                s_hi = dot16_u8(hb, x + 48, s_hi);
                float a = acc[t];
                a = __builtin_fmaf(scale[2 * p], s_lo, a);
                a = __builtin_fmaf(T == LQ_Q4_K ? scale[2 * p + 1] * 0.0625f : scale[2 * p + 1], s_hi, a);
                a = __builtin_fmaf(-minimum[2 * p], S[t][2 * p], a);
                a = __builtin_fmaf(-minimum[2 * p + 1], S[t][2 * p + 1], a);
                acc[t] = a;
            }
        }
    } else if constexpr (T == LQ_Q6_K) {
        const float d = f16_to_f32(d16);
        const uint4 scv = c[12];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const uint4 qlA = c[4 * h + jj];          // c = 0, 2 (low / high nibble)
                const uint4 qlB = c[4 * h + 2 + jj];      // c = 1, 3
                const uint4 qh = c[8 + 2 * h + jj];
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const uint4 ql = (cc & 1) ? qlB : qlA;
                    uint4 lo = (cc >= 2) ? u4_and(u4_shr(ql, 4), M0F) : u4_and(ql, M0F);
                    uint4 hi;
                    if (cc == 0) hi = u4_and(u4_shl(qh, 4), M30);
                    else if (cc == 1) hi = u4_and(u4_shl(qh, 2), M30);
                    else if (cc == 2) hi = u4_and(qh, M30);
                    else hi = u4_and(u4_shr(qh, 2), M30);
                    const uint4 q = u4_or(lo, hi);
                    const int si = 8 * h + 2 * cc + jj;        // scale / 16-group index
                    const int sbyte = si & 3;
                    const uint32_t sw = u4_get(scv, si >> 2);
                    const float ds = d * (float)(int8_t)(sw >> (8 * sbyte));
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const float *x = xs[t] + 128 * h + 32 * cc + 16 * jj;
                        float s = dot16_u8(q, x, 0.0f);
                        acc[t] = __builtin_fmaf(ds, __builtin_fmaf(-32.0f, S[t][si], s), acc[t]);
                    }
                }
            }
        }
    } else if constexpr (T == LQ_Q8_0) {
        const float d = f16_to_f32(d16);
        const uint32_t flip = 0x80808080u;   // int8 q -> q + 128 as unsigned byte
        const uint4 a = make_uint4(c[0].x ^ flip, c[0].y ^ flip, c[0].z ^ flip, c[0].w ^ flip);
        const uint4 b = make_uint4(c[1].x ^ flip, c[1].y ^ flip, c[1].z ^ flip, c[1].w ^ flip);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float s = dot16_u8(a, xs[t], 0.0f);
            s = dot16_u8(b, xs[t] + 16, s);
            acc[t] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, S[t][0], s), acc[t]);
        }
    } else if constexpr (T == LQ_Q4_0) {
        const float d = f16_to_f32(d16);
        const uint4 lo = u4_and(c[0], M0F);
        const uint4 hi = u4_and(c[0], MF0);     // 16*q
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float s = dot16_u8(lo, xs[t], 0.0f);
            s = __builtin_fmaf(0.0625f, dot16_u8(hi, xs[t] + 16, 0.0f), s);
            acc[t] = __builtin_fmaf(d, __builtin_fmaf(-8.0f, S[t][0], s), acc[t]);
        }
    }
}

// Split-K scratch of one weight handle: partial sums [ksplit][NT][tiles][64]
// and one arrival counter per tile (zero between launches).
struct SplitK {
    float *partial;
    uint32_t *counter;
    int ksplit;
};

template <int T, int NT>
__global__ __launch_bounds__(1024) void gemv_kernel(lq_geom g, const uint8_t *__restrict__ W,
                                                   const float *__restrict__ X, int64_t x_stride,
                                                   float *__restrict__ Y, int64_t y_stride, int bpw,
                                                   SplitK sk) {
    using F = Fmt<T>;
    __shared__ float red[16 * NT * 64];
    __shared__ int last;
    const int lane = lane_id();
    const int w = wave_id();
    const int nwaves = blockDim.x >> 6;
    const int tile = blockIdx.x;
    const int ks = blockIdx.y;
    const uint8_t *tbase = W + (int64_t)tile * g.tile_bytes;
    const int b0 = (ks * nwaves + w) * bpw;
    const int b1 = min((int)g.nb, b0 + bpw);

    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;

    for (int b = b0; b < b1; ++b) {
        // weights: NC coalesced 16 B loads for this block of 64 rows
        uint4 c[F::NC];
        const uint4 *src = reinterpret_cast<const uint4 *>(tbase + (int64_t)b * F::NC * 1024) + lane;
#pragma unroll
        for (int k = 0; k < F::NC; ++k) c[k] = src[64 * k];
        uint32_t d16 = 0;
        if constexpr (T == LQ_Q6_K || T == LQ_Q8_0 || T == LQ_Q4_0) {
            const uint4 dv = reinterpret_cast<const uint4 *>(tbase + g.bulk_bytes + (int64_t)(b >> 3) * 1024)[lane];
            const uint32_t dw = u4_get(dv, (b & 7) >> 1);
            d16 = (b & 1) ? (dw >> 16) : (dw & 0xffffu);
        }
        // x for this block and its group sums
        const float *xs[NT];
        float S[NT][16];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            xs[t] = X + t * x_stride + (int64_t)b * F::BV;
            if constexpr (F::BV == 256) {
                float gs = span_group_sum<F::SG>(xs[t]);
#pragma unroll
                for (int k = 0; k < 256 / F::SG; ++k) S[t][k] = uniform_f(gs, k * (F::SG / 4));
            } else {
                // 32-value block: lanes 0..7 cover it (4 values each)
                float s = 0.0f;
                if (lane < 8) {
                    const float4 v = reinterpret_cast<const float4 *>(xs[t])[lane];
                    s = (v.x + v.y) + (v.z + v.w);
                }
                S[t][0] = uniform_f(group_sum<8>(s), 0);
            }
        }
        block_dot<T, NT>(c, d16, xs, S, acc);
    }

    // workgroup partial: waves added in a fixed order
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(w * NT + t) * 64 + lane] = acc[t];
    __syncthreads();
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)tile * 64 + lane;
    float part[NT];
    int nmine = 0;
    for (int idx = tid; idx < NT * 64; idx += blockDim.x) {
        const int t = idx >> 6;
        float s = 0.0f;
        for (int k = 0; k < nwaves; ++k) s += red[(k * NT + t) * 64 + lane];
        part[nmine++] = s;
    }
    if (sk.ksplit == 1) {
        nmine = 0;
        for (int idx = tid; idx < NT * 64; idx += blockDim.x) {
            const int t = idx >> 6;
            if (row < g.rows) Y[t * y_stride + row] = part[nmine];
            ++nmine;
        }
        return;
    }
    // split-K: publish this workgroup's partial, the last arrival adds all of
    // them in ks order (deterministic) and re-arms the tile counter.
    //
    // Visibility across XCDs (each XCD has its own L2) comes from the
    // device-scope atomic accesses themselves: the partial stores and loads
    // are agent-scope atomics (device-coherent, they bypass the per-XCD L2),
    // and each wave waits for its stores to be acknowledged before the
    // workgroup counts its arrival. An agent-scope fence would do the same
    // with a full L2 write-back + invalidate per workgroup, which measured
    // ~12x slower for the whole kernel.
    nmine = 0;
    for (int idx = tid; idx < NT * 64; idx += blockDim.x) {
        const int t = idx >> 6;
        float *dst = sk.partial + (((int64_t)ks * NT + t) * g.tiles + tile) * 64 + lane;
        __hip_atomic_store(dst, part[nmine++], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        uint32_t old = __hip_atomic_fetch_add(sk.counter + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (old == (uint32_t)sk.ksplit - 1);
    }
    __syncthreads();
    if (!last) return;
    for (int idx = tid; idx < NT * 64; idx += blockDim.x) {
        const int t = idx >> 6;
        float s = 0.0f;
        for (int k = 0; k < sk.ksplit; ++k) {
            const float *p = sk.partial + (((int64_t)k * NT + t) * g.tiles + tile) * 64 + lane;
            s += __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (row < g.rows) Y[t * y_stride + row] = s;
    }
    if (tid == 0) __hip_atomic_store(sk.counter + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch plan. A workgroup owns one 64-row tile and splits its K range over
// up to 16 waves (partials added in LDS). Matrices with fewer tiles than
// ~192 also split K across workgroups, just enough to give ~256 workgroups
// (one per CU): the cross-workgroup combine costs a few memory round trips,
// so it is only worth it when CUs would otherwise sit idle.
GemvPlan gemv_plan(const lq_geom &g) {
    GemvPlan p;
    int64_t ksplit = 1;
    if (g.tiles < 192) {
        ksplit = (256 + g.tiles - 1) / g.tiles;
        if (ksplit > g.nb) ksplit = g.nb;
    }
    int64_t per_wg = (g.nb + ksplit - 1) / ksplit;          // blocks per workgroup
    int64_t waves = per_wg < 16 ? per_wg : 16;
    int64_t bpw = (per_wg + waves - 1) / waves;
    waves = (per_wg + bpw - 1) / bpw;
    ksplit = (g.nb + waves * bpw - 1) / (waves * bpw);
    p.waves = (int)waves;
    p.bpw = (int)bpw;
    p.ksplit = (int)ksplit;
    return p;
}

template <int T>
static int launch_t(const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y,
                    int64_t ys, int ntok, float *partial, uint32_t *counter, hipStream_t s) {
    const GemvPlan p = gemv_plan(g);
    for (int t0 = 0; t0 < ntok; t0 += 8) {
        int nt = ntok - t0 < 8 ? ntok - t0 : 8;
        const float *xp = x + t0 * xs;
        float *yp = y + t0 * ys;
        dim3 grid((unsigned)g.tiles, (unsigned)p.ksplit), block(64 * p.waves);
        SplitK sk{partial, counter, p.ksplit};
        switch (nt) {
#define LQ_GV(N) case N: hipLaunchKernelGGL((gemv_kernel<T, N>), grid, block, 0, s, g, W, xp, xs, yp, ys, p.bpw, sk); break;
            LQ_GV(1) LQ_GV(2) LQ_GV(3) LQ_GV(4) LQ_GV(5) LQ_GV(6) LQ_GV(7) LQ_GV(8)
#undef LQ_GV
        }
        LQ_HIP(hipGetLastError());
    }
    return LOCALAI_OK;
}

int launch_matvec(const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y,
                  int64_t ys, int ntok, float *partial, uint32_t *counter, hipStream_t s) {
    if (reinterpret_cast<uintptr_t>(x) & 15 || (xs & 3))
        return fail(LOCALAI_EARG, "matvec x must be 16-byte aligned with a row stride multiple of 4");
    if (gemv_plan(g).ksplit > 1 && (!partial || !counter))
        return fail(LOCALAI_EARG, "matvec: split-K scratch missing");
    switch (g.type) {
        case LQ_Q4_K: return launch_t<LQ_Q4_K>(g, W, x, xs, y, ys, ntok, partial, counter, s);
        case LQ_Q5_K: return launch_t<LQ_Q5_K>(g, W, x, xs, y, ys, ntok, partial, counter, s);
        case LQ_Q6_K: return launch_t<LQ_Q6_K>(g, W, x, xs, y, ys, ntok, partial, counter, s);
        case LQ_Q8_0: return launch_t<LQ_Q8_0>(g, W, x, xs, y, ys, ntok, partial, counter, s);
        case LQ_Q4_0: return launch_t<LQ_Q4_0>(g, W, x, xs, y, ys, ntok, partial, counter, s);
        default: return fail(LOCALAI_ETYPE, "matvec: unsupported GGML type");
    }
}

}  // namespace lq
