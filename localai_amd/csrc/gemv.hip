// Dense decode matvec: y[t, r] = sum_c W[r, c] * x[t, c] for t < ntok.
// Mapping and arithmetic: gemv_core.h.
//
// Launch plan: a workgroup owns a tile of consecutive rows and all of K. Rows
// of more than 32 units (K > 2048) get 64 lanes per row and ceil(U / 64)
// waves that split K (S = 2 units per lane per wave beyond 16384 values,
// keeping a workgroup at 4 waves up to K = 32768); shorter rows get 32 or 16
// lanes per row and one wave. Each wave holds its x windows (16 KiB per
// 64-unit slot and vector) in LDS; vector pairs are used up to K = 8192. No state crosses
// workgroups, so a launch is one round trip of loads per wave plus the
// in-wave and LDS reductions, and any matrix size yields rows / tile
// workgroups.
#include "gemv_core.h"
#include "internal.h"

namespace lq {

// rows per lane group: 8 for one vector (processed 2 per pipeline step), 4
// for two vectors, 2 with two unit slots
template <int T, int NT, int S>
constexpr int rows_per_lane() {
    return S == 2 ? 2 : NT == 2 ? 4 : 8;
}
template <int T, int NT, int S>
constexpr int rows_per_step() {
    return S == 2 ? 2 : 2;
}

template <int T, int NT, int S, int LPR>
__global__ __launch_bounds__(256) void gemv_kernel(lq_geom g, const uint8_t *__restrict__ W,
                                                   const float *__restrict__ X, int64_t x_stride,
                                                   float *__restrict__ Y, int64_t y_stride) {
    constexpr int R = rows_per_lane<T, NT, S>();
    constexpr int G = 64 / LPR;
    extern __shared__ float4 xlds[];   // S * NT * 16 * LPR float4 per wave
    __shared__ float red[4 * R * NT];
    const int w = wave_id(), nw = blockDim.x >> 6;
    const int64_t row0 = (int64_t)blockIdx.x * R * G;
    const float *xrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xrow[t] = X + t * x_stride;
    int vi;
    bool writer;
    const float part = wave_rows<T, NT, S, R, LPR, 1, rows_per_step<T, NT, S>()>(
        W, g, row0, 0, g.rows, w * S, xrow, xlds + w * S * NT * 16 * LPR, vi, writer);
    if (nw == 1) {
        const int r = vi / NT, t = vi % NT;
        const int64_t row = row0 + (lane_id() / LPR) * R + r;
        if (writer && row < g.rows) Y[t * y_stride + row] = part;
        return;
    }
    // several waves: LPR == 64, one row group
    if (writer) red[w * R * NT + vi] = part;
    __syncthreads();
    const int i = threadIdx.x;
    if (i < R * NT) {
        float s = 0.0f;
        for (int k = 0; k < nw; ++k) s += red[k * R * NT + i];
        const int r = i / NT, t = i % NT;
        if (row0 + r < g.rows) Y[t * y_stride + row0 + r] = s;
    }
}

GemvPlan gemv_plan(const lq_geom &g, int nt) {
    GemvPlan p;
    const int64_t U = g.nu;
    p.lpr = lanes_per_row(U);
    p.slots = U > 256 ? 2 : 1;
    p.waves = p.lpr < 64 ? 1 : (int)((U + 64 * p.slots - 1) / (64 * p.slots));
    const int r = p.slots == 2 ? 2 : nt == 2 ? 4 : 8;
    p.rows = r * (64 / p.lpr);
    p.lds_bytes = (size_t)p.waves * p.slots * nt * 16 * p.lpr * 16;
    return p;
}

template <int T, int NT, int S, int LPR>
static void launch_k(const GemvPlan &p, const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y,
                     int64_t ys, hipStream_t s) {
    dim3 grid((unsigned)((g.rows + p.rows - 1) / p.rows)), block(64 * p.waves);
    hipLaunchKernelGGL((gemv_kernel<T, NT, S, LPR>), grid, block, p.lds_bytes, s, g, W, x, xs, y, ys);
}

template <int T, int NT>
static int launch_nt(const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y, int64_t ys,
                     hipStream_t s) {
    const GemvPlan p = gemv_plan(g, NT);
    if (p.waves > 4) return fail(LOCALAI_EARG, "matvec: K too large (more than 32768 values per row)");
    if (p.lds_bytes > max_lds_per_block()) return fail(LOCALAI_EARG, "matvec: x window exceeds the LDS per workgroup");
    if (p.lpr == 16) launch_k<T, NT, 1, 16>(p, g, W, x, xs, y, ys, s);
    else if (p.lpr == 32) launch_k<T, NT, 1, 32>(p, g, W, x, xs, y, ys, s);
    else if (p.slots == 1) launch_k<T, NT, 1, 64>(p, g, W, x, xs, y, ys, s);
    else if constexpr (NT == 1) launch_k<T, 1, 2, 64>(p, g, W, x, xs, y, ys, s);
    else return fail(LOCALAI_EARG, "matvec: vector pairs need K <= 16384");
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

template <int T>
static int launch_t(const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y, int64_t ys,
                    int ntok, hipStream_t s) {
    const bool pairs = g.nu <= 128;   // two x windows per wave within 64 KiB of LDS
    for (int t0 = 0; t0 < ntok;) {
        const int nt = (pairs && ntok - t0 >= 2) ? 2 : 1;
        int st = nt == 2 ? launch_nt<T, 2>(g, W, x + t0 * xs, xs, y + t0 * ys, ys, s)
                         : launch_nt<T, 1>(g, W, x + t0 * xs, xs, y + t0 * ys, ys, s);
        if (st) return st;
        t0 += nt;
    }
    return LOCALAI_OK;
}

int launch_matvec(const lq_geom &g, const uint8_t *W, const float *x, int64_t xs, float *y, int64_t ys,
                  int ntok, hipStream_t s) {
    if (reinterpret_cast<uintptr_t>(x) & 15 || (xs & 3))
        return fail(LOCALAI_EARG, "matvec x must be 16-byte aligned with a row stride multiple of 4");
    if (g.cols % 32) return fail(LOCALAI_EARG, "matvec: cols must be a multiple of 32");
    switch (g.type) {
        case LQ_Q4_K: return launch_t<LQ_Q4_K>(g, W, x, xs, y, ys, ntok, s);
        case LQ_Q5_K: return launch_t<LQ_Q5_K>(g, W, x, xs, y, ys, ntok, s);
        case LQ_Q6_K: return launch_t<LQ_Q6_K>(g, W, x, xs, y, ys, ntok, s);
        case LQ_Q8_0: return launch_t<LQ_Q8_0>(g, W, x, xs, y, ys, ntok, s);
        case LQ_Q4_0: return launch_t<LQ_Q4_0>(g, W, x, xs, y, ys, ntok, s);
        default: return fail(LOCALAI_ETYPE, "matvec: unsupported GGML type");
    }
}

}  // namespace lq
