// fp32 matrix times vectors: y[t, r] = sum_c W[r, c] * x[t, c], t < ntok.
//
// The device path for GGUF tensors outside the packed types (F32, F16, Q4_1,
// Q5_0, Q5_1 matrices): the reference decodes them to fp32 and runs
// `weights @ x` in NumPy (engine/gguf_parser.py:269-289, :350-358); here the
// dequant kernels decode once into a device fp32 matrix and this kernel reads
// it. HBM-bound: each row is read once per call (4 cols bytes), the vectors
// come from L2.
//
// One wave per row, four rows per workgroup. Lane l sums elements 4l + 256j
// (+0..3) in j order, then the 64 partials meet in a fixed xor tree, so a
// result does not depend on the launch. Up to 4 tokens per pass share one
// read of the row.
#include "dev_common.h"
#include "internal.h"

namespace lq {

constexpr int DN_TOK = 4;

template <bool VEC>
__global__ __launch_bounds__(256) void f32_matvec_kernel(const float *__restrict__ W, int64_t rows, int64_t cols,
                                                         const float *__restrict__ X, int64_t ntok,
                                                         float *__restrict__ Y) {
    const int lane = lane_id();
    const int64_t r = (int64_t)blockIdx.x * 4 + wave_id();
    if (r >= rows) return;
    const float *w = W + r * cols;
    for (int64_t t0 = 0; t0 < ntok; t0 += DN_TOK) {
        const int nt = (int)(ntok - t0 < DN_TOK ? ntok - t0 : DN_TOK);
        float s[DN_TOK] = {0.f, 0.f, 0.f, 0.f};
        if (VEC) {
            for (int64_t c = 4 * lane; c < cols; c += 256) {
                const float4 wv = *reinterpret_cast<const float4 *>(w + c);
#pragma unroll
                for (int i = 0; i < DN_TOK; ++i) {
                    if (i < nt) {
                        const float4 xv = *reinterpret_cast<const float4 *>(X + (t0 + i) * cols + c);
                        s[i] = __builtin_fmaf(wv.x, xv.x, s[i]);
                        s[i] = __builtin_fmaf(wv.y, xv.y, s[i]);
                        s[i] = __builtin_fmaf(wv.z, xv.z, s[i]);
                        s[i] = __builtin_fmaf(wv.w, xv.w, s[i]);
                    }
                }
            }
        } else {
            for (int64_t c = lane; c < cols; c += 64) {
                const float wv = w[c];
#pragma unroll
                for (int i = 0; i < DN_TOK; ++i)
                    if (i < nt) s[i] = __builtin_fmaf(wv, X[(t0 + i) * cols + c], s[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < DN_TOK; ++i) {
            float v = s[i];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0 && i < nt) Y[(t0 + i) * rows + r] = v;
        }
    }
}

int launch_f32_matvec(const float *W, int64_t rows, int64_t cols, const float *x, int64_t ntok, float *y,
                      hipStream_t s) {
    if (rows < 1 || cols < 1 || ntok < 1) return fail(LOCALAI_EARG, "f32 matvec: rows, cols and tokens must be >= 1");
    if (rows > ((int64_t)1 << 32)) return fail(LOCALAI_EARG, "f32 matvec: too many rows");
    const bool vec = cols % 4 == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (vec)
        hipLaunchKernelGGL(f32_matvec_kernel<true>, grid, dim3(256), 0, s, W, rows, cols, x, ntok, y);
    else
        hipLaunchKernelGGL(f32_matvec_kernel<false>, grid, dim3(256), 0, s, W, rows, cols, x, ntok, y);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
