// Device code of the decode matvec ("row-split" mapping), shared by the
// dense matvec (gemv.hip) and the grouped MoE matvecs (moe.hip).
//
// A row of K values is cut into 64-value units (qformat.h). A lane owns one
// unit of a row at a time; LPR consecutive lanes (64, or 32 / 16 for rows of
// at most 32 / 16 units) cover a slice of LPR units of one row, so a wave
// works on 64 / LPR rows at once and R row steps. With LPR = 64 a workgroup
// has ceil(U / 64) waves, wave w owning units 64w .. 64w + 63 (S = 2 slots of
// 64 units per wave beyond 8 waves' worth). The unit's 64 x values stay in
// VGPRs and are reused for every row the wave visits; they reach the lanes
// through LDS so that both the HBM weight loads and the x loads are
// coalesced 1 KiB per instruction. Per-row partial sums are added across the
// LPR lanes with a transposed butterfly (R rows x NT vectors reduced
// together), and across waves through LDS in a fixed order.
//
// Arithmetic: fp32 products of exactly decoded integer quants with fp32 x,
// fp32 accumulation; block and sub-block scales are applied once per unit,
// like the factorisation of engine/native_quant.cpp:183-337 (without
// quantising x):
//   Q4_K/Q5_K  (d*sc_g) * sum q*x - (dmin*mn_g) * sum x     per 32-value group
//   Q6_K       (d*sc_s) * (sum q6*x - 32 * sum x)           per 16-value sub-block
//   Q8_0       d * (sum (q+128)*x - 128 * sum x)
//   Q4_0       d * (sum q4*x - 8 * sum x)
// 4-bit codes are converted with v_cvt_pk_f32_fp8: read as fp8 e4m3 the byte
// 0000qqqq is exactly q * 2^-9 (subnormal for q < 8, exponent 1 above), so
// one instruction converts two nibbles; the 2^9 goes into the scale.
#pragma once
#include "dev_common.h"

namespace lq {

typedef float lq_float2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
// 16 bytes read once (nontemporal hint)
__device__ __forceinline__ uint4 ld16_nt(const uint8_t *p) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v t = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

// sum_i code_i * x[i] over the 16 nibble codes in q (bytes 0..15, each < 16),
// codes decoded as fp8 e4m3 = code * 2^-9
__device__ __forceinline__ float dot16_fp8(uint4 q, const float *x) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = u4_get(q, d);
        const lq_float2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
        const lq_float2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
        a0 = __builtin_fmaf(lo.x, x[4 * d + 0], a0);
        a1 = __builtin_fmaf(lo.y, x[4 * d + 1], a1);
        a0 = __builtin_fmaf(hi.x, x[4 * d + 2], a0);
        a1 = __builtin_fmaf(hi.y, x[4 * d + 3], a1);
    }
    return a0 + a1;
}

// sum_i byte_i * x[i] over the 16 unsigned bytes of q
__device__ __forceinline__ float dot16_u8(uint4 q, const float *x) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = u4_get(q, d);
        a0 = __builtin_fmaf(ubyte0(w), x[4 * d + 0], a0);
        a1 = __builtin_fmaf(ubyte1(w), x[4 * d + 1], a1);
        a0 = __builtin_fmaf(ubyte2(w), x[4 * d + 2], a0);
        a1 = __builtin_fmaf(ubyte3(w), x[4 * d + 3], a1);
    }
    return a0 + a1;
}

__device__ __forceinline__ uint4 u4_and(uint4 a, uint32_t m) { return make_uint4(a.x & m, a.y & m, a.z & m, a.w & m); }
__device__ __forceinline__ uint4 u4_shr(uint4 a, uint32_t s) { return make_uint4(a.x >> s, a.y >> s, a.z >> s, a.w >> s); }
__device__ __forceinline__ uint4 u4_shl(uint4 a, uint32_t s) { return make_uint4(a.x << s, a.y << s, a.z << s, a.w << s); }
__device__ __forceinline__ uint4 u4_or(uint4 a, uint4 b) { return make_uint4(a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w); }
__device__ __forceinline__ uint4 u4_xor(uint4 a, uint32_t m) { return make_uint4(a.x ^ m, a.y ^ m, a.z ^ m, a.w ^ m); }

// ---------------------------------------------------------------------------
// x staging. A wave's x window is the x range of its 64-unit slot (4096
// values, fewer at the row end). Unit order of a unit's 64 values:
//   Q6_K    xr[16c + e] = value 128h + 32c + 16m + e of the super-block
//   others  the unit's 64 consecutive values
// In LDS, float4 q (0..15) of local unit i sits at slot 16i + (q ^ (i & 15)):
// the 16 lanes of a quarter-wave read 16 different 16-byte bank groups.

// A window's x loads: LPR / 4 float4 per lane (load k of lane l is window
// float4 64k + l, so each load instruction reads 1 KiB contiguous). Float4s
// at or past nq (the row end) read as zero.
template <int LPR>
__device__ __forceinline__ void stage_load(const float *__restrict__ xw, int nq, float4 *v) {
    const float4 *p = reinterpret_cast<const float4 *>(xw);
    const int lane = lane_id();
#pragma unroll
    for (int k = 0; k < LPR / 4; ++k) {
        const int f = 64 * k + lane;
        const float4 t = p[f < nq ? f : nq - 1];
        v[k] = f < nq ? t : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// Store the loaded window into LDS in unit order, then wait for the writes:
// the lanes that read a unit's x are not the lanes that wrote it.
template <int T, int LPR>
__device__ __forceinline__ void stage_store(float4 *lds, const float4 *v) {
    const int lane = lane_id();
#pragma unroll
    for (int k = 0; k < LPR / 4; ++k) {
        const int f = 64 * k + lane;
        int i, q;
        if constexpr (T == LQ_Q6_K) {
            const int fl = f & 63;   // 32h + 8c + 4m + e/4 inside the super-block
            i = 4 * (f >> 6) + 2 * (fl >> 5) + ((fl >> 2) & 1);
            q = 4 * ((fl >> 3) & 3) + (fl & 3);
        } else {
            i = f >> 4;
            q = f & 15;
        }
        lds[16 * i + (q ^ (i & 15))] = v[k];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ void stage_read(const float4 *lds, int i, float *xr) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float4 t = lds[16 * i + (q ^ (i & 15))];
        xr[4 * q + 0] = t.x; xr[4 * q + 1] = t.y; xr[4 * q + 2] = t.z; xr[4 * q + 3] = t.w;
    }
}

// Sums of the four 16-value quarters of a unit's x values (unit order).
__device__ __forceinline__ void quarter_sums(const float *xr, float *q4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += xr[16 * q + i];
        q4[q] = s;
    }
}

// ---------------------------------------------------------------------------
// Weight fields of one unit of one row, loaded ahead of the arithmetic.
struct UnitW {
    uint4 q0, q1, q2, q3;   // quant pieces
    uint4 h0, h1;           // K-quant header; Q6_K qh in h0; Q5_K qh in h1, q2
    uint32_t sc;            // Q6_K scales (4 x int8); Q8_0/Q4_0 d pair
    uint32_t d;             // Q6_K d
};

// Unit u of a row; C = units in u's 64-unit chunk (qformat.h interleave).
template <int T>
__device__ __forceinline__ UnitW load_unit_w(const uint8_t *__restrict__ W, const lq_geom &g, int64_t row, int u,
                                             int C) {
    UnitW w;
    const uint8_t *p0 = W + g.plane[0] + row * g.pitch[0];
    const uint8_t *p1 = W + g.plane[1] + row * g.pitch[1];
    const int c0 = u & ~63, i = u - c0;
    if constexpr (T == LQ_Q4_K) {
        w.q0 = ld16_nt(p0 + 16 * (2 * c0 + i));
        w.q1 = ld16_nt(p0 + 16 * (2 * c0 + C + i));
        w.h0 = ld16(p1 + 16 * (u >> 2));
    } else if constexpr (T == LQ_Q5_K) {
        const uint8_t *p2 = W + g.plane[2] + row * g.pitch[2];
        const int sb = u >> 2, s0 = c0 >> 2, cs = C >> 2;
        w.q0 = ld16_nt(p0 + 16 * (2 * c0 + i));
        w.q1 = ld16_nt(p0 + 16 * (2 * c0 + C + i));
        w.h1 = ld16(p1 + 16 * (2 * s0 + (sb - s0)));        // qh[0..15]
        w.q2 = ld16_nt(p1 + 16 * (2 * s0 + cs + (sb - s0)));   // qh[16..31]
        w.h0 = ld16(p2 + 16 * sb);
    } else if constexpr (T == LQ_Q6_K) {
        const uint8_t *p2 = W + g.plane[2] + row * g.pitch[2];
        const uint8_t *p3 = W + g.plane[3] + row * g.pitch[3];
        w.q0 = ld16_nt(p0 + 16 * (2 * c0 + i));                // ql[16m .. 16m+15] of half h
        w.q1 = ld16_nt(p0 + 16 * (2 * c0 + C + i));            // ql[32+16m ..]
        w.h0 = ld16(p1 + 16 * u);                           // qh[16m ..] of half h
        w.sc = ld4(p2 + 4 * u);
        w.d = *reinterpret_cast<const uint16_t *>(p3 + 2 * (u >> 2));
    } else if constexpr (T == LQ_Q8_0) {
        w.q0 = ld16_nt(p0 + 16 * (4 * c0 + i));
        w.q1 = ld16_nt(p0 + 16 * (4 * c0 + C + i));
        w.q2 = ld16_nt(p0 + 16 * (4 * c0 + 2 * C + i));
        w.q3 = ld16_nt(p0 + 16 * (4 * c0 + 3 * C + i));
        w.sc = ld4(p1 + 4 * u);
    } else {   // Q4_0
        w.q0 = ld16_nt(p0 + 16 * (2 * c0 + i));
        w.q1 = ld16_nt(p0 + 16 * (2 * c0 + C + i));
        w.sc = ld4(p1 + 4 * u);
    }
    return w;
}

// K-quant 6-bit (scale, min) of groups 2p and 2p+1 from the 16-byte header h.
// Branch-free: p varies across lanes, and a select written as ?: is turned
// into divergent branches by the compiler.
__device__ __forceinline__ void kq_pair(uint4 h, int p, uint32_t &sc0, uint32_t &sc1, uint32_t &mn0,
                                        uint32_t &mn1) {
    const uint32_t upper = 0u - (uint32_t)(p >> 1);          // all ones for groups 4..7
    const uint32_t sc_a = h.y & 0x3F3F3F3Fu;
    const uint32_t mn_a = h.z & 0x3F3F3F3Fu;
    const uint32_t sc_b = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t mn_b = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    const uint32_t sh = 16u * (uint32_t)(p & 1);
    const uint32_t scw = ((sc_a & ~upper) | (sc_b & upper)) >> sh;
    const uint32_t mnw = ((mn_a & ~upper) | (mn_b & upper)) >> sh;
    sc0 = scw & 0xFFu;
    sc1 = (scw >> 8) & 0xFFu;
    mn0 = mnw & 0xFFu;
    mn1 = (mnw >> 8) & 0xFFu;
}

// Contribution of unit u (weights w, x values xr in unit order, quarter sums
// q4) to one row.
template <int T>
__device__ __forceinline__ float unit_dot(const UnitW &w, int u, const float *xr, const float *q4) {
    const uint32_t M0F = opaque(0x0F0F0F0Fu);
    if constexpr (T == LQ_Q4_K) {
        uint32_t sc0, sc1, mn0, mn1;
        kq_pair(w.h0, u & 3, sc0, sc1, mn0, mn1);
        const float d = f16_to_f32(w.h0.x) * 512.0f, dmin = f16_to_f32(w.h0.x >> 16);
        const float slo = dot16_fp8(u4_and(w.q0, M0F), xr) + dot16_fp8(u4_and(w.q1, M0F), xr + 16);
        const float shi = dot16_fp8(u4_and(u4_shr(w.q0, 4), M0F), xr + 32) +
                          dot16_fp8(u4_and(u4_shr(w.q1, 4), M0F), xr + 48);
        float r = (d * (float)sc0) * slo;
        r = __builtin_fmaf(d * (float)sc1, shi, r);
        r = __builtin_fmaf(-dmin * (float)mn0, q4[0] + q4[1], r);
        return __builtin_fmaf(-dmin * (float)mn1, q4[2] + q4[3], r);
    } else if constexpr (T == LQ_Q5_K) {
        const int p = u & 3;
        uint32_t sc0, sc1, mn0, mn1;
        kq_pair(w.h0, p, sc0, sc1, mn0, mn1);
        const float d = f16_to_f32(w.h0.x), dmin = f16_to_f32(w.h0.x >> 16);
        const uint32_t g0 = 2 * p, g1 = 2 * p + 1;
        const uint32_t B1 = opaque(0x01010101u);
        const uint4 l0 = u4_or(u4_and(w.q0, M0F), u4_shl(u4_and(u4_shr(w.h1, g0), B1), 4));
        const uint4 l1 = u4_or(u4_and(w.q1, M0F), u4_shl(u4_and(u4_shr(w.q2, g0), B1), 4));
        const uint4 h0 = u4_or(u4_and(u4_shr(w.q0, 4), M0F), u4_shl(u4_and(u4_shr(w.h1, g1), B1), 4));
        const uint4 h1 = u4_or(u4_and(u4_shr(w.q1, 4), M0F), u4_shl(u4_and(u4_shr(w.q2, g1), B1), 4));
        float r = (d * (float)sc0) * (dot16_u8(l0, xr) + dot16_u8(l1, xr + 16));
        r = __builtin_fmaf(d * (float)sc1, dot16_u8(h0, xr + 32) + dot16_u8(h1, xr + 48), r);
        r = __builtin_fmaf(-dmin * (float)mn0, q4[0] + q4[1], r);
        return __builtin_fmaf(-dmin * (float)mn1, q4[2] + q4[3], r);
    } else if constexpr (T == LQ_Q6_K) {
        // quad c: low nibbles of ql[l] (c = 0, 2 from q0) or ql[l+32] (c = 1, 3
        // from q1), high nibble for c >= 2; 2 high bits at qh bits 2c, 2c+1
        const uint32_t M30 = opaque(0x30303030u);
        const uint4 a0 = u4_or(u4_and(w.q0, M0F), u4_and(u4_shl(w.h0, 4), M30));
        const uint4 a1 = u4_or(u4_and(w.q1, M0F), u4_and(u4_shl(w.h0, 2), M30));
        const uint4 a2 = u4_or(u4_and(u4_shr(w.q0, 4), M0F), u4_and(w.h0, M30));
        const uint4 a3 = u4_or(u4_and(u4_shr(w.q1, 4), M0F), u4_and(u4_shr(w.h0, 2), M30));
        const float d = f16_to_f32(w.d);
        float r = (float)(int8_t)w.sc * __builtin_fmaf(-32.0f, q4[0], dot16_u8(a0, xr));
        r = __builtin_fmaf((float)(int8_t)(w.sc >> 8), __builtin_fmaf(-32.0f, q4[1], dot16_u8(a1, xr + 16)), r);
        r = __builtin_fmaf((float)(int8_t)(w.sc >> 16), __builtin_fmaf(-32.0f, q4[2], dot16_u8(a2, xr + 32)), r);
        r = __builtin_fmaf((float)(int8_t)(w.sc >> 24), __builtin_fmaf(-32.0f, q4[3], dot16_u8(a3, xr + 48)), r);
        return d * r;
    } else if constexpr (T == LQ_Q8_0) {
        const uint32_t flip = 0x80808080u;   // int8 q -> q + 128 as an unsigned byte
        const float s0 = dot16_u8(u4_xor(w.q0, flip), xr) + dot16_u8(u4_xor(w.q1, flip), xr + 16);
        const float s1 = dot16_u8(u4_xor(w.q2, flip), xr + 32) + dot16_u8(u4_xor(w.q3, flip), xr + 48);
        const float r = f16_to_f32(w.sc) * __builtin_fmaf(-128.0f, q4[0] + q4[1], s0);
        return __builtin_fmaf(f16_to_f32(w.sc >> 16), __builtin_fmaf(-128.0f, q4[2] + q4[3], s1), r);
    } else {   // Q4_0: block 2u low/high nibbles = values 0..15 / 16..31, block 2u+1 likewise
        const float s0 = 512.0f * (dot16_fp8(u4_and(w.q0, M0F), xr) + dot16_fp8(u4_and(u4_shr(w.q0, 4), M0F), xr + 16));
        const float s1 = 512.0f * (dot16_fp8(u4_and(w.q1, M0F), xr + 32) + dot16_fp8(u4_and(u4_shr(w.q1, 4), M0F), xr + 48));
        const float r = f16_to_f32(w.sc) * __builtin_fmaf(-8.0f, q4[0] + q4[1], s0);
        return __builtin_fmaf(f16_to_f32(w.sc >> 16), __builtin_fmaf(-8.0f, q4[2] + q4[3], s1), r);
    }
}

// Transposed butterfly inside groups of LPR lanes: N values per lane
// (N <= LPR, powers of two) become one sum per value; lanes whose index in the
// group is a multiple of LPR / N hold the total of value `index`.
template <int N, int LPR>
__device__ __forceinline__ float xreduce(float *v, int &index) {
    const int lane = lane_id();
    int idx = 0;
    int m = LPR / 2;
#pragma unroll
    for (int n = N; n > 1; n >>= 1, m >>= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < n / 2; ++i) {
            const float keep = upper ? v[i + n / 2] : v[i];
            const float send = upper ? v[i] : v[i + n / 2];
            v[i] = keep + __shfl_xor(send, m, 64);
        }
        if (upper) idx += n / 2;
    }
    float s = v[0];
#pragma unroll
    for (; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    index = idx;
    return s;
}

// Lanes per row for rows of U units: 64, or 32 / 16 when the row is that short.
__host__ __device__ __forceinline__ int lanes_per_row(int64_t U) { return U <= 16 ? 16 : U <= 32 ? 32 : 64; }

// Rows: lane group gi = lane / LPR (G = 64 / LPR groups) takes rows
// set_base + gi * RG + rr, rr < RG = R / SETS, of each of the SETS row sets
// (set 0 starts at row0, set 1 at rowb); rows >= nrows contribute zero.
// Units: slot s of the wave covers units 64 * (slot0 + s) + (lane % LPR).
// lds: this wave's S * NT * 16 * LPR float4 of LDS. xrow[t]: vector t (K floats).
// The R rows are processed P at a time (R / P steps) with the weight fields
// of the next two steps in flight: step i + 2 is issued once step i's
// arithmetic is done, so each wave streams its rows while it computes
// instead of waiting for all of them and computing at the end.
// Returns, for writer lanes, the partial sum over this wave's units of value
// vi = r * NT + t (r = set * RG + rr) of the lane's group.
template <int T, int NT, int S, int R, int LPR, int SETS = 1, int P = R>
__device__ __forceinline__ float wave_rows(const uint8_t *__restrict__ W, const lq_geom &g, int64_t row0,
                                           int64_t rowb, int64_t nrows, int slot0,
                                           const float *const *xrow, float4 *lds, int &vi, bool &writer) {
    static_assert(R % SETS == 0 && R * NT <= LPR && R % P == 0, "row map");
    constexpr int STEPS = R / P;
    const int lane = lane_id();
    const int U = (int)g.nu;
    const int gi = lane / LPR, li = lane % LPR;
    constexpr int RG = R / SETS;
    // x windows are loaded first, then the first two steps' weight fields,
    // with no arithmetic in between (scheduler barrier); loads complete in
    // issue order, so the LDS transposition of x waits only for the x loads.
    float4 xs[S][NT][LPR / 4];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t v0 = (int64_t)64 * 64 * (slot0 + s);
        int64_t nq = (g.cols - v0) / 4;
        nq = nq < 16 * LPR ? nq : 16 * LPR;
        nq = nq > 1 ? nq : 1;
        const int64_t vc = v0 < g.cols ? v0 : 0;
#pragma unroll
        for (int t = 0; t < NT; ++t) stage_load<LPR>(xrow[t] + vc, (int)nq, xs[s][t]);
    }
    UnitW wt[2][P][S];
    bool live[2][P][S];
    auto issue = [&](int buf, int step) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int r = step * P + p;
            const int set = r / RG, rr = r % RG;
            const int64_t want = (set ? rowb : row0) + gi * RG + rr;
            const bool row_live = want < nrows;
            const int64_t row = row_live ? want : nrows - 1;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int u = 64 * (slot0 + s) + li;
                const int uc = u < U ? u : U - 1;
                const int c0 = uc & ~63;
                const int C = U - c0 < 64 ? U - c0 : 64;
                live[buf][p][s] = u < U && row_live;
                wt[buf][p][s] = load_unit_w<T>(W, g, row, uc, C);
            }
        }
    };
    issue(0, 0);
    if (STEPS > 1) issue(1, 1);
    __builtin_amdgcn_sched_barrier(0);
    float xr[S][NT][64], q4[S][NT][4];
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float4 *region = lds + (s * NT + t) * 16 * LPR;
            stage_store<T, LPR>(region, xs[s][t]);
            stage_read(region, li, xr[s][t]);
            quarter_sums(xr[s][t], q4[s][t]);
        }
    }
    float acc[R * NT];
#pragma unroll
    for (int i = 0; i < R * NT; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
        const int buf = st & 1;
#pragma unroll
        for (int p = 0; p < P; ++p) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int u = 64 * (slot0 + s) + li;
                const int uc = u < U ? u : U - 1;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float c = unit_dot<T>(wt[buf][p][s], uc, xr[s][t], q4[s][t]);
                    acc[(st * P + p) * NT + t] += live[buf][p][s] ? c : 0.0f;
                }
            }
        }
        if (st + 2 < STEPS) {
            __builtin_amdgcn_sched_barrier(0);
            issue(buf, st + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const float total = xreduce<R * NT, LPR>(acc, vi);
    writer = (li & (LPR / (R * NT) - 1)) == 0;
    return total;
}

}  // namespace lq
