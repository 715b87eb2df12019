// ZAYA's MoE router and expert epilogues on the device
// (engine/zaya.py:274-307).
//
// The router of one token is an MLP on a 256-wide state (each projection
// plus its GGUF bias when the file has one, engine/model.py:72-79):
//   r     = W_inp h                       (a matvec launch: gguf matrix)
//   r     = r + prev * eda                 EDA from the previous MoE layer
//   state = r                              returned to the caller
//   u     = rmsnorm(r) * w_norm
//   v1    = gelu(W_gate u), v2 = gelu(W_mlp2 v1), logits = W_mlp4 v2
//   probs = softmax(logits), expert = argmax(probs + bias)  (first maximum)
// zaya_router_tail_kernel runs everything after W_inp in one workgroup: the
// three small matrices (fp32 device copies) are read once, every vector
// stays in LDS. The expert index and the probabilities are written for the
// host, which picks the expert tensors (or the skip route) to run next.
//
// Arithmetic follows the reference's fp32 NumPy steps where the rounding is
// fixed by them: the EDA product and sum, the RMSNorm products, the softmax
// subtraction and division, and the bias addition are separate fp32
// operations (no fused multiply-add); exact GELU takes math.erf in fp64 and
// multiplies in fp32, as NumPy >= 2 does for a float32 scalar; the sums of
// the matvecs, of the norm and of the softmax are fp64 in a fixed order,
// rounded once (NumPy sums fp32 pairwise, so these can differ in the last
// bit; the exponential is the device's expf, NumPy's is its own).
#include "dev_common.h"
#include "internal.h"

namespace lq {

constexpr int ZR_THREADS = 1024;
constexpr int ZR_MAXV = 4096;   // largest vector of the router MLP

// y[i] = sum_c W[i, c] x[c] (fp64, lanes then a fixed tree), one row per wave
// at a time; W [rows, cols] fp32 in device memory, x / y in LDS
__device__ __forceinline__ void zr_matvec(const float *__restrict__ W, const float *__restrict__ b, int rows,
                                          int cols, const float *x, float *y, bool gelu) {
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    for (int i = w; i < rows; i += nw) {
        const float *row = W + (int64_t)i * cols;
        double s = 0.0;
        for (int c = lane; c < cols; c += 64) s = __builtin_fma((double)row[c], (double)x[c], s);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) {
            float v = (float)s;
            if (b) v = __fadd_rn(v, b[i]);
            if (gelu) {
                // v * (1 + erf(v / sqrt 2)) * 0.5 with the bracket computed in
                // fp64 and the products in fp32 (a NumPy float32 scalar times a
                // Python float stays float32, NumPy >= 2)
                const float b = (float)(1.0 + erf((double)v / 1.4142135623730951));
                v = __fmul_rn(__fmul_rn(v, b), 0.5f);
            }
            y[i] = v;
        }
    }
    __syncthreads();
}

// Block sum of a per-thread fp64 value (fixed order: waves, then lanes of a tree)
__device__ __forceinline__ double zr_block_sum(double v, double *red) {
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int k = 0; k < nw; ++k) s += red[k];
    __syncthreads();
    return s;
}

__global__ __launch_bounds__(ZR_THREADS) void zaya_router_tail_kernel(
    const float *__restrict__ r0, const float *__restrict__ b0, const float *__restrict__ prev,
    const float *__restrict__ eda, const float *__restrict__ norm_w, float eps, int R, const float *__restrict__ W1,
    const float *__restrict__ b1, int R1, const float *__restrict__ W2, const float *__restrict__ b2, int R2,
    const float *__restrict__ W3, const float *__restrict__ b3, int NE, const float *__restrict__ bias,
    float *__restrict__ state, float *__restrict__ probs, int32_t *__restrict__ expert,
    float *__restrict__ expert_w) {
    __shared__ float va[ZR_MAXV], vb[ZR_MAXV];
    __shared__ double red[ZR_THREADS / 64];
    const int t = threadIdx.x;
    // EDA and the norm's mean square
    double sq = 0.0;
    for (int i = t; i < R; i += blockDim.x) {
        float r = r0[i];
        if (b0) r = __fadd_rn(r, b0[i]);
        if (prev) r = __fadd_rn(r, __fmul_rn(prev[i], eda[i]));
        state[i] = r;
        va[i] = r;
        sq += (double)r * (double)r;
    }
    const double ms = zr_block_sum(sq, red);
    // x * (1 / sqrt(mean(x * x) + eps)) * w in fp32 steps
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)(ms / (double)R), eps)));
    for (int i = t; i < R; i += blockDim.x) vb[i] = __fmul_rn(__fmul_rn(va[i], inv), norm_w[i]);
    __syncthreads();
    zr_matvec(W1, b1, R1, R, vb, va, true);     // v1 = gelu(W_gate u + b1)
    zr_matvec(W2, b2, R2, R1, va, vb, true);    // v2 = gelu(W_mlp2 v1 + b2)
    zr_matvec(W3, b3, NE, R2, vb, va, false);   // logits = W_mlp4 v2 + b3
    // softmax over NE logits (one wave; NE <= 64 * 8), then argmax(probs + bias)
    if (t < 64) {
        float m = -INFINITY;
        for (int i = t; i < NE; i += 64) m = fmaxf(m, va[i]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        double z = 0.0;
        for (int i = t; i < NE; i += 64) {
            const float e = expf(__fsub_rn(va[i], m));
            vb[i] = e;
            z += (double)e;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);
        const float zf = (float)z;
        float best = -INFINITY;
        int bi = NE;
        for (int i = t; i < NE; i += 64) {
            const float p = __fdiv_rn(vb[i], zf);
            probs[i] = p;
            const float route = __fadd_rn(p, bias[i]);
            if (route > best || (route == best && i < bi)) {
                best = route;
                bi = i;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
        if (t == 0) {
            const int e = bi < NE ? bi : 0;
            expert[0] = e;
            // the chosen route's probability, the same division as probs[e]
            // (vb was written by this wave)
            if (expert_w) expert_w[0] = __fdiv_rn(vb[e], zf);
        }
    }
}

int launch_zaya_router_tail(const float *r0, const float *b0, const float *prev, const float *eda,
                            const float *norm_w, float eps, int R, const float *W1, const float *b1, int R1,
                            const float *W2, const float *b2, int R2, const float *W3, const float *b3, int NE,
                            const float *bias, float *state, float *probs, int32_t *expert, float *expert_w,
                            hipStream_t s) {
    if (R < 1 || R1 < 1 || R2 < 1 || NE < 1 || R > ZR_MAXV || R1 > ZR_MAXV || R2 > ZR_MAXV || NE > 512)
        return fail(LOCALAI_EARG, "zaya router: vector sizes 1..4096, at most 512 routes");
    if ((prev == nullptr) != (eda == nullptr)) return fail(LOCALAI_EARG, "zaya router: prev and eda go together");
    hipLaunchKernelGGL(zaya_router_tail_kernel, dim3(1), dim3(ZR_THREADS), 0, s, r0, b0, prev, eda, norm_w, eps, R,
                       W1, b1, R1, W2, b2, R2, W3, b3, NE, bias, state, probs, expert, expert_w);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

// gu != null: y[i] = silu(gu[i]) * gu[n + i], the expert's SwiGLU on the
// [gate; up] output of gate_up (engine/zaya.py:304-305); gu == null:
// y[i] = x[i] * scale[0], the route probability applied to the expert output
// or to h for the skip route (:297-301, :306). scale is device memory (the
// router's probs), so the host need not read it.
__global__ void zaya_scale_kernel(const float *__restrict__ gu, const float *__restrict__ x, int64_t n,
                                  const float *__restrict__ scale, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (gu) {
        const float g = gu[i];
        // g / (1 + exp(-clip(g, -80, 80))) in fp32 steps
        const float gc = fminf(fmaxf(g, -80.0f), 80.0f);
        const float sl = __fdiv_rn(g, __fadd_rn(1.0f, expf(-gc)));
        y[i] = __fmul_rn(sl, gu[n + i]);
    } else {
        y[i] = __fmul_rn(x[i], scale[0]);
    }
}

int launch_zaya_scale(const float *gu, const float *x, int64_t n, const float *scale, float *y, hipStream_t s) {
    if (n < 1) return fail(LOCALAI_EARG, "zaya scale: n >= 1");
    if (!gu && (!x || !scale)) return fail(LOCALAI_EARG, "zaya scale: x and scale, or gu");
    hipLaunchKernelGGL(zaya_scale_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, x, n, scale, y);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
