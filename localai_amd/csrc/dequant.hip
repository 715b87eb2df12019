// Dequantisation straight from GGML bytes (engine/dequant.py:27-167).
//
// One thread decodes 8 consecutive values of one block and writes them with
// two 16-byte stores, so a wave writes 2 KiB contiguous. Source bytes are read
// with byte loads: GGML blocks of 18/22/34/210 bytes are only 2-byte aligned
// and the reads are a small fraction of the traffic (0.56-1.06 B in per 4 B
// out). Arithmetic is float32 in the reference's association, so every value
// is bit-identical to engine/dequant.py / engine/native_quant.cpp:543-618:
// all products are exact and the affine types round once at the final add.
#include "dev_common.h"
#include "ggml_decode.h"
#include "internal.h"

namespace lq {

template <int T>
__global__ void dequant_kernel(const uint8_t *__restrict__ raw, int64_t nvals, float *__restrict__ out) {
    constexpr int BV = T == LQ_Q4_K || T == LQ_Q5_K || T == LQ_Q6_K ? 256 : 32;
    constexpr int BPB = T == LQ_Q4_0 ? 18 : T == LQ_Q4_1 ? 20 : T == LQ_Q5_0 ? 22 : T == LQ_Q5_1 ? 24
                      : T == LQ_Q8_0 ? 34 : T == LQ_Q4_K ? 144 : T == LQ_Q5_K ? 176 : 210;
    const int64_t n8 = nvals / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t e = i * 8;
        int64_t b = e / BV;
        float v[8];
        decode8<T>(raw + b * BPB, (int)(e - b * BV), v);
        float4 *o = reinterpret_cast<float4 *>(out + e);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// F32 / F16: element-wise (engine/dequant.py:39-42).
__global__ void dequant_f16_kernel(const uint16_t *__restrict__ raw, int64_t n, float *__restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f16_to_f32_bits(raw[i]);
}

int launch_dequant_ggml(int t, const void *raw, int64_t n, float *out, hipStream_t s) {
    if (n <= 0) return LOCALAI_OK;
    if (t == LQ_F32) {
        LQ_HIP(hipMemcpyAsync(out, raw, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
        return LOCALAI_OK;
    }
    if (t == LQ_F16) {
        if (reinterpret_cast<uintptr_t>(raw) & 1) return fail(LOCALAI_EARG, "F16 source must be 2-byte aligned");
        int64_t blocks = (n + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(dequant_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           (const uint16_t *)raw, n, out);
        LQ_HIP(hipGetLastError());
        return LOCALAI_OK;
    }
    if (reinterpret_cast<uintptr_t>(out) & 15)
        return fail(LOCALAI_EARG, "dequant output must be 16-byte aligned");
    int64_t blocks = (n / 8 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    const uint8_t *r = (const uint8_t *)raw;
    switch (t) {
#define LQ_DQ(T)                                                                        \
    case T:                                                                             \
        hipLaunchKernelGGL(dequant_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, r, n, out); \
        break;
        LQ_DQ(LQ_Q4_0) LQ_DQ(LQ_Q4_1) LQ_DQ(LQ_Q5_0) LQ_DQ(LQ_Q5_1) LQ_DQ(LQ_Q8_0)
        LQ_DQ(LQ_Q4_K) LQ_DQ(LQ_Q5_K) LQ_DQ(LQ_Q6_K)
#undef LQ_DQ
        default: return fail(LOCALAI_ETYPE, "unsupported GGML type for dequant");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// Largest row L2 norm of each row half of every matrix: one wave per row
// sums the squares of its exact decoded values in fp64; lane 0 rounds the
// norm up to a float and raises the matrix's half (out[2 b + (row >=
// rows / 2)]) to it with an unsigned atomic max (non-negative floats order
// like their bits; NaN, bits above inf, wins). The MoE gate_up GEMM bounds
// its SiLU * up outputs with these.
template <int T>
__global__ __launch_bounds__(256) void row_norm_kernel(const uint8_t *__restrict__ raw, int64_t rows, int64_t cols,
                                                       int64_t nrows, float *__restrict__ out) {
    constexpr int BV = T == LQ_Q4_K || T == LQ_Q5_K || T == LQ_Q6_K ? 256 : 32;
    constexpr int BPB = T == LQ_Q4_0 ? 18 : T == LQ_Q4_1 ? 20 : T == LQ_Q5_0 ? 22 : T == LQ_Q5_1 ? 24
                      : T == LQ_Q8_0 ? 34 : T == LQ_Q4_K ? 144 : T == LQ_Q5_K ? 176 : 210;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= nrows) return;
    const int lane = threadIdx.x & 63;
    const uint8_t *row = raw + r * (cols / BV) * BPB;
    double ss = 0.0;
    for (int64_t e = 8 * lane; e < cols; e += 512) {
        float v[8];
        decode8<T>(row + (e / BV) * BPB, (int)(e % BV), v);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) {
        const float f = (float)sqrt(ss);   // >= 0 or NaN
        // the next float up (one more in the bits of a non-negative float)
        const unsigned up = __builtin_bit_cast(unsigned, f) + (f < __builtin_inff() ? 1u : 0u);
        const int64_t rr = r % rows;
        atomicMax(reinterpret_cast<unsigned *>(out) + 2 * (r / rows) + (rr >= rows / 2 ? 1 : 0),
                  up);
    }
}

int launch_row_norms(const lq_geom &g, const uint8_t *ggml, float *out, hipStream_t s) {
    LQ_HIP(hipMemsetAsync(out, 0, (size_t)(2 * g.batch) * sizeof(float), s));
    const int64_t nrows = g.rows * g.batch;
    const dim3 grid((unsigned)((nrows + 3) / 4));
    switch (g.type) {
#define LQ_RN(T)                                                                                                 \
    case T:                                                                                                      \
        hipLaunchKernelGGL(row_norm_kernel<T>, grid, dim3(256), 0, s, ggml, g.rows, g.cols, nrows, out);         \
        break;
        LQ_RN(LQ_Q4_0) LQ_RN(LQ_Q8_0) LQ_RN(LQ_Q4_K) LQ_RN(LQ_Q5_K) LQ_RN(LQ_Q6_K)
#undef LQ_RN
        default: return fail(LOCALAI_ETYPE, "row norms: unsupported type");
    }
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
