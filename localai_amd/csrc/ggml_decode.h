// Exact decoders of GGML blocks from their bytes (engine/dequant.py:27-167),
// shared by the dequant kernels and the matvec that reads GGML bytes.
// Arithmetic is float32 in the reference's association, so every value is
// bit-identical to engine/dequant.py / engine/native_quant.cpp:543-618: all
// products are exact and the affine types round once at the final add.
// Bytes are read one at a time (GGML's 18/22/34/210-byte blocks are only
// 2-byte aligned).
#pragma once
#include "dev_common.h"

namespace lq {

__device__ __forceinline__ uint32_t rd8(const uint8_t *p, int off) { return p[off]; }
__device__ __forceinline__ uint32_t rd16(const uint8_t *p, int off) {
    return (uint32_t)p[off] | ((uint32_t)p[off + 1] << 8);
}

// K-quant 6-bit scale/min of group g from the 12-byte table at `s`
// (engine/native_quant.cpp:117-124).
__device__ __forceinline__ uint32_t kq_scale(const uint8_t *s, int g) {
    return g < 4 ? (s[g] & 63u) : ((s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4));
}
__device__ __forceinline__ uint32_t kq_min(const uint8_t *s, int g) {
    return g < 4 ? (s[g + 4] & 63u) : ((uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4));
}

// Decode values e0..e0+7 of the block at `blk`.
template <int T>
__device__ __forceinline__ void decode8(const uint8_t *__restrict__ blk, int e0, float v[8]) {
    if constexpr (T == LQ_Q8_0) {
        const float d = f16_to_f32_bits(rd16(blk, 0));
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)blk[2 + e0 + i] * d;
    } else if constexpr (T == LQ_Q4_0 || T == LQ_Q4_1) {
        const float d = f16_to_f32_bits(rd16(blk, 0));
        const int qo = T == LQ_Q4_0 ? 2 : 4;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int e = e0 + i;
            uint32_t q = (blk[qo + (e & 15)] >> (4 * (e >> 4))) & 15u;
            if constexpr (T == LQ_Q4_0) v[i] = ((float)q - 8.0f) * d;
            else v[i] = __builtin_fmaf((float)q, d, f16_to_f32_bits(rd16(blk, 2)));
        }
    } else if constexpr (T == LQ_Q5_0 || T == LQ_Q5_1) {
        const float d = f16_to_f32_bits(rd16(blk, 0));
        const int ho = T == LQ_Q5_0 ? 2 : 4;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int e = e0 + i;
            uint32_t lo = (blk[ho + 4 + (e & 15)] >> (4 * (e >> 4))) & 15u;
            uint32_t hi = (blk[ho + (e >> 3)] >> (e & 7)) & 1u;
            float q = (float)(lo | (hi << 4));
            if constexpr (T == LQ_Q5_0) v[i] = (q - 16.0f) * d;
            else v[i] = __builtin_fmaf(q, d, f16_to_f32_bits(rd16(blk, 2)));
        }
    } else if constexpr (T == LQ_Q4_K || T == LQ_Q5_K) {
        const float d = f16_to_f32_bits(rd16(blk, 0));
        const float dmin = f16_to_f32_bits(rd16(blk, 2));
        const int g = e0 >> 5, j0 = e0 & 31;
        const float scale = d * (float)kq_scale(blk + 4, g);
        const float minimum = dmin * (float)kq_min(blk + 4, g);
        const uint8_t *qs = blk + (T == LQ_Q4_K ? 16 : 48) + 32 * (g >> 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t q = (qs[j0 + i] >> (4 * (g & 1))) & 15u;
            if constexpr (T == LQ_Q5_K) q |= ((blk[16 + j0 + i] >> g) & 1u) << 4;
            // (d*sc)*q is exact, so the fused form rounds once like scale*q - minimum.
            v[i] = __builtin_fmaf((float)q, scale, -minimum);
        }
    } else if constexpr (T == LQ_Q6_K) {
        const float d = f16_to_f32_bits(rd16(blk, 208));
        const int h = e0 >> 7, c = (e0 >> 5) & 3, j0 = e0 & 31;
        const float ds = d * (float)(int8_t)blk[192 + 8 * h + 2 * c + (j0 >> 4)];
        const uint8_t *ql = blk + 64 * h + 32 * (c & 1);
        const uint8_t *qh = blk + 128 + 32 * h;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t lo = (ql[j0 + i] >> (4 * (c >> 1))) & 15u;
            uint32_t hi = (qh[j0 + i] >> (2 * c)) & 3u;
            v[i] = ds * (float)((int)(lo | (hi << 4)) - 32);
        }
    }
}

}  // namespace lq
