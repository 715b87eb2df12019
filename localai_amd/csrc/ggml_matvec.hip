// Matvec straight from GGML bytes kept on the device, for the types without
// a tile or row-planes form: F16, Q4_1, Q5_0, Q5_1 (F32, Q4_0 and Q8_0 are
// accepted too). y[t, r] = sum_c W[r, c] * x[t, c] for t < ntok.
//
// The reference decodes such matrices to fp32 (or fp16) and multiplies in
// NumPy (engine/gguf_parser.py:269-289, :350-358, its matrix caches at
// :65-69). Here the device holds the file's bytes as they are -- F16 2 B per
// value instead of 4, Q4_1 / Q5_0 / Q5_1 0.63 to 0.75 B -- and each wave
// decodes its row's blocks in registers with the exact formulas of
// engine/dequant.py (ggml_decode.h: every decoded value is bit-identical to
// the reference's) before its fp32 products. HBM-bound: the row's bytes once
// per pass of up to four tokens.
//
// One wave per row, four rows per workgroup. Lane l takes the 8-value groups
// l, l + 64, ... of the row (the four groups of a 32-value block fall on
// adjacent lanes, so a wave's byte reads of one pass are contiguous), sums
// them in that order, and the 64 partials meet in a fixed xor tree: results
// do not depend on the launch.
#include "dev_common.h"
#include "ggml_decode.h"
#include "internal.h"

namespace lq {

constexpr int GV_TOK = 4;

template <int T>
__device__ __forceinline__ void gv_group(const uint8_t *__restrict__ w, int64_t g, float v[8]) {
    if constexpr (T == LQ_F32) {
        const float4 a = reinterpret_cast<const float4 *>(w)[2 * g], b = reinterpret_cast<const float4 *>(w)[2 * g + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else if constexpr (T == LQ_F16) {
        const uint4 h = reinterpret_cast<const uint4 *>(w)[g];
        const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = f16_to_f32_bits(hw[i] & 0xFFFFu);
            v[2 * i + 1] = f16_to_f32_bits(hw[i] >> 16);
        }
    } else {
        constexpr int BPB = T == LQ_Q4_0 ? 18 : T == LQ_Q4_1 ? 20 : T == LQ_Q5_0 ? 22 : T == LQ_Q5_1 ? 24 : 34;
        decode8<T>(w + (g >> 2) * BPB, (int)(g & 3) * 8, v);
    }
}

// cols % 8 == 0; X rows and W rows (F32 / F16) 16-byte aligned
template <int T>
__global__ __launch_bounds__(256) void ggml_matvec_kernel(const uint8_t *__restrict__ W, int64_t rows, int64_t cols,
                                                          int64_t row_bytes, const float *__restrict__ X,
                                                          int64_t ntok, float *__restrict__ Y) {
    const int lane = lane_id();
    const int64_t r = (int64_t)blockIdx.x * 4 + wave_id();
    if (r >= rows) return;
    const uint8_t *w = W + r * row_bytes;
    const int64_t ng = cols >> 3;
    for (int64_t t0 = 0; t0 < ntok; t0 += GV_TOK) {
        const int nt = (int)(ntok - t0 < GV_TOK ? ntok - t0 : GV_TOK);
        float s[GV_TOK] = {0.f, 0.f, 0.f, 0.f};
        for (int64_t g = lane; g < ng; g += 64) {
            float v[8];
            gv_group<T>(w, g, v);
#pragma unroll
            for (int i = 0; i < GV_TOK; ++i) {
                if (i < nt) {
                    const float4 *xp = reinterpret_cast<const float4 *>(X + (t0 + i) * cols) + 2 * g;
                    const float4 a = xp[0], b = xp[1];
                    s[i] = __builtin_fmaf(v[0], a.x, s[i]);
                    s[i] = __builtin_fmaf(v[1], a.y, s[i]);
                    s[i] = __builtin_fmaf(v[2], a.z, s[i]);
                    s[i] = __builtin_fmaf(v[3], a.w, s[i]);
                    s[i] = __builtin_fmaf(v[4], b.x, s[i]);
                    s[i] = __builtin_fmaf(v[5], b.y, s[i]);
                    s[i] = __builtin_fmaf(v[6], b.z, s[i]);
                    s[i] = __builtin_fmaf(v[7], b.w, s[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < GV_TOK; ++i) {
            float v = s[i];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0 && i < nt) Y[(t0 + i) * rows + r] = v;
        }
    }
}

int launch_ggml_matvec(int t, const void *W, int64_t rows, int64_t cols, const float *x, int64_t ntok, float *y,
                       hipStream_t s) {
    if (rows < 1 || cols < 1 || ntok < 1) return fail(LOCALAI_EARG, "ggml matvec: rows, cols and tokens must be >= 1");
    if (rows > ((int64_t)1 << 32)) return fail(LOCALAI_EARG, "ggml matvec: too many rows");
    const int bv = lq_block_values(t);
    if (cols % 8 || cols % bv) return fail(LOCALAI_EARG, "ggml matvec: cols must be a multiple of 8 and of the block size");
    const int64_t row_bytes = cols / bv * lq_block_bytes(t);
    if ((uintptr_t)x & 15) return fail(LOCALAI_EARG, "ggml matvec: x must be 16-byte aligned");
    if ((t == LQ_F32 || t == LQ_F16) && ((uintptr_t)W & 15))
        return fail(LOCALAI_EARG, "ggml matvec: F32 / F16 weights must be 16-byte aligned");
    const dim3 grid((unsigned)((rows + 3) / 4));
    const uint8_t *w = (const uint8_t *)W;
    switch (t) {
#define LQ_GV(TT)                                                                                            \
    case TT:                                                                                                 \
        hipLaunchKernelGGL(ggml_matvec_kernel<TT>, grid, dim3(256), 0, s, w, rows, cols, row_bytes, x, ntok, y); \
        break;
        LQ_GV(LQ_F32) LQ_GV(LQ_F16) LQ_GV(LQ_Q4_0) LQ_GV(LQ_Q4_1) LQ_GV(LQ_Q5_0) LQ_GV(LQ_Q5_1) LQ_GV(LQ_Q8_0)
#undef LQ_GV
        default: return fail(LOCALAI_ETYPE, "ggml matvec: F32, F16, Q4_0, Q4_1, Q5_0, Q5_1 or Q8_0");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
