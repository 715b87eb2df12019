// Streaming-read kernel: the HBM read floor that the decode kernels are
// measured against (bench.py's hbm_read_floor workload). It reads `bytes`
// (a multiple of 16) once, 16 bytes per lane per load, each wave keeping two
// groups of U loads in flight over a grid-stride walk, and folds the data
// into one word so the loads cannot be dropped.
#include "dev_common.h"
#include "internal.h"

namespace lq {

constexpr int SR_U = 2;          // 1 KiB loads per wave per group
constexpr int SR_THREADS = 1024;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const uint4 *__restrict__ p, int64_t n16,
                                                                 uint32_t *__restrict__ out) {
    const int64_t nw = (int64_t)gridDim.x * (SR_THREADS / 64);
    const int64_t w = (int64_t)blockIdx.x * (SR_THREADS / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t ngroups = n16 / (64 * SR_U);   // whole groups; the rest below
    uint32_t acc = 0;
    uint4 a[SR_U], b[SR_U];
    auto ld = [&](uint4 (&v)[SR_U], int64_t g) {
        g = g < ngroups ? g : ngroups - 1;
#pragma unroll
        for (int u = 0; u < SR_U; ++u) v[u] = p[(g * SR_U + u) * 64 + lane];
    };
    auto fold = [&](const uint4 (&v)[SR_U]) {
#pragma unroll
        for (int u = 0; u < SR_U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    };
    if (ngroups > 0 && w < ngroups) {
        ld(a, w);
        for (int64_t g = w; g < ngroups; g += 2 * nw) {
            ld(b, g + nw);
            fold(a);
            ld(a, g + 2 * nw);
            if (g + nw < ngroups) fold(b);
        }
    }
    // tail: the 16-byte words past the last whole group, one per thread
    for (int64_t i = ngroups * SR_U * 64 + w * 64 + lane; i < n16; i += nw * 64) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[0] = acc;   // practically never: the loads stay live
}

int launch_stream_read(const void *src, int64_t bytes, uint32_t *out, hipStream_t s) {
    int dev = 0, cus = 0;
    LQ_HIP(hipGetDevice(&dev));
    LQ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t n16 = bytes / 16;
    if (n16 <= 0) return LOCALAI_OK;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)(2 * cus)), dim3(SR_THREADS), 0, s,
                       (const uint4 *)src, n16, out);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
