// GGML <-> row-planes repack (a lossless byte permutation plus zero padding,
// layout in qformat.h).
#include "dev_common.h"
#include "internal.h"

namespace lq {

// Calls f(plane, offset inside the plane row, GGML offset inside the row or
// -1 for zero padding, length) for every field piece owned by unit u.
// Shared per-super-block fields are owned by the super-block's first unit.
template <class F>
__device__ __forceinline__ void unit_moves(const lq_geom &g, int64_t u, F f) {
    const int64_t U = g.nu, nb = g.nb;
    switch (g.type) {
        case LQ_Q4_K: {
            const int64_t sb = u >> 2, p = u & 3, base = sb * 144;
            for (int j = 0; j < 2; ++j) f(0, lq_ilv(u, U, 2, j, 64), base + 16 + 32 * p + 16 * j, 16);
            if (p == 0) f(1, 16 * sb, base, 16);
            break;
        }
        case LQ_Q5_K: {
            const int64_t sb = u >> 2, p = u & 3, base = sb * 176;
            for (int j = 0; j < 2; ++j) f(0, lq_ilv(u, U, 2, j, 64), base + 48 + 32 * p + 16 * j, 16);
            if (p == 0) {
                for (int j = 0; j < 2; ++j) f(1, lq_ilv(sb, nb, 2, j, 16), base + 16 + 16 * j, 16);
                f(2, 16 * sb, base, 16);
            }
            break;
        }
        case LQ_Q6_K: {
            const int64_t sb = u >> 2, h = (u >> 1) & 1, m = u & 1, base = sb * 210;
            for (int j = 0; j < 2; ++j) f(0, lq_ilv(u, U, 2, j, 64), base + 64 * h + 16 * m + 32 * j, 16);
            f(1, 16 * u, base + 128 + 32 * h + 16 * m, 16);
            for (int c = 0; c < 4; ++c) f(2, 4 * u + c, base + 192 + 8 * h + m + 2 * c, 1);
            if ((u & 3) == 0) f(3, 2 * sb, base + 208, 2);
            break;
        }
        case LQ_Q8_0: {
            for (int j = 0; j < 4; ++j) {
                const int64_t b = 2 * u + (j >> 1);
                f(0, lq_ilv(u, U, 4, j, 64), b < nb ? b * 34 + 2 + 16 * (j & 1) : -1, 16);
            }
            for (int i = 0; i < 2; ++i) {
                const int64_t b = 2 * u + i;
                f(1, 4 * u + 2 * i, b < nb ? b * 34 : -1, 2);
            }
            break;
        }
        case LQ_Q4_0: {
            for (int j = 0; j < 2; ++j) {
                const int64_t b = 2 * u + j;
                f(0, lq_ilv(u, U, 2, j, 64), b < nb ? b * 18 + 2 : -1, 16);
            }
            for (int i = 0; i < 2; ++i) {
                const int64_t b = 2 * u + i;
                f(1, 4 * u + 2 * i, b < nb ? b * 18 : -1, 2);
            }
            break;
        }
        default: break;
    }
}

// direction 0: ggml -> planes (padding written as zeros); 1: planes -> ggml.
// One thread per (matrix, row, unit); byte copies, since GGML blocks are only
// 2-byte aligned and the repack runs once per weight upload.
__global__ void repack_kernel(lq_geom g, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int direction) {
    const int64_t total = g.batch * g.rows * g.nu;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * g.nu);
        const int64_t rem = i - e * g.rows * g.nu;
        const int64_t row = rem / g.nu;
        const int64_t u = rem - row * g.nu;
        const int64_t grow = e * g.ggml_matrix_bytes + row * g.ggml_row_bytes;
        unit_moves(g, u, [&](int p, int64_t pofs, int64_t gofs, int len) {
            const int64_t prow = e * g.matrix_bytes + g.plane[p] + row * g.pitch[p] + pofs;
            if (direction == 0) {
                for (int k = 0; k < len; ++k) dst[prow + k] = gofs >= 0 ? src[grow + gofs + k] : 0;
            } else if (gofs >= 0) {
                for (int k = 0; k < len; ++k) dst[grow + gofs + k] = src[prow + k];
            }
        });
    }
}

int launch_repack(const lq_geom &g, const uint8_t *src, uint8_t *dst, int direction, hipStream_t s) {
    const int64_t total = g.batch * g.rows * g.nu;
    if (total <= 0) return LOCALAI_OK;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, src, dst, direction);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
