// f16 rows of activations for the MFMA GEMMs: one wave converts one token
// row (x_to_f16_row), called by the conversion kernels of gemm.hip and by
// the MoE top-k kernel, whose waves each own one token anyway.
#pragma once
#include "dev_common.h"

namespace lq {

// Row t (one wave) reads X row src = rows_map ? rows_map[t] / k : t and writes
//   Xh[t, 0..ldh) = f16(X[src, c] * 2^s) (zero past cols),  inv[t] = 2^-s,
// with 2^s bringing the row's largest finite magnitude into [2^14, 2^15)
// (s = 0 for an all-zero or non-finite maximum). Lanes move 8-value groups
// (two 16-byte loads, one 16-byte store); NG > 0: the lane's NG groups stay
// in registers between the max and the conversion, NG = 0: the row is read
// twice. cols is a multiple of 8; vec: X rows are 16-byte aligned.
// tiled: Xh holds MFMA A operands instead of rows: token t's values
// 32 q + 8 c .. + 7 (c < 4) go to 16-byte slot ((t / 16) * (ldh / 32) + q) * 64
// + (t % 16) + 16 c, so that one 32-value slice of 16 tokens is 1 KB
// contiguous in lane order; tokens ntok .. ntok_pad - 1 are written as zeros.
// nrm2 (not null): nrm2[t] = the row's sum of squares (fp32; NaN or inf
// where the row holds one).
template <int NG>
__device__ __forceinline__ void x_to_f16_row(int64_t t, const float *__restrict__ X, int64_t ldx, int cols,
                                             const int32_t *__restrict__ rows_map, int k, int64_t ntok,
                                             _Float16 *__restrict__ Xh, int ldh, float *__restrict__ inv, int vec,
                                             int tiled, int64_t ntok_pad, float *__restrict__ nrm2 = nullptr) {
    const int lane = lane_id();
    if (t >= ntok_pad) return;
    if (t >= ntok) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int gi = lane; gi < (ldh >> 3); gi += 64)
            *reinterpret_cast<h8 *>(Xh + 8 * ((((t >> 4) * (ldh >> 5) + (gi >> 2)) << 6) + (t & 15) + 16 * (gi & 3))) = z;
        return;
    }
    const int64_t src = rows_map ? (int64_t)(rows_map[t] / k) : t;
    const float *x = X + src * ldx;
    const int ngx = cols >> 3, ng = ldh >> 3;
    auto load = [&](int gi, lq_f4 &lo, lq_f4 &hi) {
        if (vec) {
            lo = *reinterpret_cast<const lq_f4 *>(x + 8 * gi);
            hi = *reinterpret_cast<const lq_f4 *>(x + 8 * gi + 4);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                lo[c] = x[8 * gi + c];
                hi[c] = x[8 * gi + 4 + c];
            }
        }
    };
    // the largest magnitude as ordered bits; NaN counts as zero (fmaxf's rule)
    auto mag = [](const lq_f4 &v) {
        uint32_t m = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float f = v[c];   // bit_cast of a vector element would read element 0
            const uint32_t u = __builtin_bit_cast(uint32_t, f) & 0x7fffffffu;
            m = max(m, u > 0x7f800000u ? 0u : u);
        }
        return m;
    };
    auto sq = [](const lq_f4 &v) { return v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]; };
    constexpr int NR = NG > 0 ? NG : 1;
    lq_f4 lo[NR], hi[NR];
    uint32_t mb = 0;
    float ss = 0.0f;
    if (NG > 0) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int gi = lane + 64 * i;
            lo[i] = hi[i] = lq_f4{0.f, 0.f, 0.f, 0.f};
            if (gi < ngx) load(gi, lo[i], hi[i]);
        }
#pragma unroll
        for (int i = 0; i < NR; ++i) mb = max(mb, max(mag(lo[i]), mag(hi[i])));
        if (nrm2)
#pragma unroll
            for (int i = 0; i < NR; ++i) ss += sq(lo[i]) + sq(hi[i]);
    } else {
        for (int gi = lane; gi < ngx; gi += 64) {
            lq_f4 l, h;
            load(gi, l, h);
            mb = max(mb, max(mag(l), mag(h)));
            if (nrm2) ss += sq(l) + sq(h);
        }
    }
    if (nrm2) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) nrm2[t] = ss;
    }
    const float m = __builtin_bit_cast(float, wave_max_u32(mb));
    int s = 0;
    if (m > 0.0f && m <= 3.4e38f) {
        int e;
        frexpf(m, &e);          // m < 2^e <= 2m
        s = 15 - e;             // m * 2^s in [2^14, 2^15)
        s = s > 120 ? 120 : s < -120 ? -120 : s;
    }
    const float sc = ldexpf(1.0f, s);   // exact power of two: x * sc == ldexpf(x, s) in the f16 range
    _Float16 *xh = Xh + t * ldh;
    auto store = [&](int gi, const lq_f4 &l, const lq_f4 &h) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            o[c] = (_Float16)(l[c] * sc);
            o[4 + c] = (_Float16)(h[c] * sc);
        }
        if (tiled)
            *reinterpret_cast<h8 *>(Xh + 8 * ((((t >> 4) * (ldh >> 5) + (gi >> 2)) << 6) + (t & 15) + 16 * (gi & 3))) = o;
        else
            *reinterpret_cast<h8 *>(xh + 8 * gi) = o;
    };
    if (NG > 0) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int gi = lane + 64 * i;
            if (gi < ng) store(gi, lo[i], hi[i]);
        }
    } else {
        for (int gi = lane; gi < ng; gi += 64) {
            lq_f4 l = {0.f, 0.f, 0.f, 0.f}, h = l;
            if (gi < ngx) load(gi, l, h);
            store(gi, l, h);
        }
    }
    if (lane == 0) inv[t] = ldexpf(1.0f, -s);
}

}  // namespace lq
