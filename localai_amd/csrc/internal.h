// Internal interfaces shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "qformat.h"
#include "../../include/localai_hip.h"

struct localai_qmat {
    lq_geom g;
    uint8_t *data;      // device, g.matrix_bytes * g.batch
    float *partial;     // split-K partial sums of the matvec, [ksplit][8][tiles][64]
    uint32_t *counter;  // one arrival counter per row-tile, zero between launches
    int device;
};

namespace lq {

// Error state (thread-local), set by the entry points.
int fail(int status, const std::string &msg);
int hip_fail(hipError_t e, const char *what);
void clear_error();
void set_legacy_status(int status);

#define LQ_HIP(expr)                                      \
    do {                                                  \
        hipError_t _e = (expr);                           \
        if (_e != hipSuccess) return lq::hip_fail(_e, #expr); \
    } while (0)

int ensure_device();   // make the library's device current for this thread

// launchers (return LOCALAI_* status)
int launch_repack(const lq_geom &g, const uint8_t *ggml, uint8_t *packed, int direction,
                  hipStream_t s);
int launch_dequant_ggml(int t, const void *raw, int64_t n, float *out, hipStream_t s);
int launch_dequant_packed(const lq_geom &g, const uint8_t *packed, float *out, hipStream_t s);
struct GemvPlan {
    int waves;    // waves per workgroup
    int bpw;      // blocks per wave
    int ksplit;   // workgroups sharing one row-tile (K split)
};
GemvPlan gemv_plan(const lq_geom &g);
int launch_matvec(const lq_geom &g, const uint8_t *packed, const float *x, int64_t x_stride,
                  float *y, int64_t y_stride, int ntok, float *partial, uint32_t *counter,
                  hipStream_t s);

}  // namespace lq
