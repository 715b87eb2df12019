// Streaming-read kernel: the HBM read floor that the decode kernels are
// measured against (bench.py's hbm_read_floor workload). It reads `bytes`
// (a multiple of 16) once, 16 bytes per lane per load with the nontemporal
// hint (the decode kernels' weight loads carry it too), over a grid-stride
// walk of 4 workgroups of 512 threads per CU, and folds the data into one
// word so the loads cannot be dropped. Of the launch shapes and load kinds
// swept on MI355X (256 to 4096 workgroups of 256 to 1024 threads, one, two or
// four loads in flight per lane, plain or nontemporal), this one read the
// decode layer's bytes fastest both as its four launches and as one.
#include "dev_common.h"
#include "internal.h"

namespace lq {

constexpr int SR_THREADS = 512;
constexpr int SR_PER_CU = 4;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const uint4 *__restrict__ p, int64_t n16,
                                                                 uint32_t *__restrict__ out) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const u4 *q = reinterpret_cast<const u4 *>(p);
    const int64_t stride = (int64_t)gridDim.x * SR_THREADS;
    uint32_t acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * SR_THREADS + threadIdx.x; i < n16; i += stride) {
        const u4 v = __builtin_nontemporal_load(q + i);
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
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)(SR_PER_CU * cus)), dim3(SR_THREADS), 0, s,
                       (const uint4 *)src, n16, out);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
