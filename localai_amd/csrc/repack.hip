// GGML <-> lane-interleaved repack (a lossless byte permutation, see qformat.h).
#include "dev_common.h"
#include "internal.h"

namespace lq {

// direction 0: ggml -> packed (padding rows written as zero); 1: packed -> ggml.
// One thread moves one 16-byte bulk chunk or one 8-block group of fp16 scales.
__global__ void repack_kernel(lq_geom g, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int direction) {
    const int t = g.type;
    const int nchunk = lq_nchunk(t);
    const int bpb = lq_block_bytes(t);
    const int64_t ngroup = lq_has_d16(t) ? (g.nb + 7) / 8 : 0;
    const int64_t bulk_items = g.nb * nchunk * 64;
    const int64_t items_per_tile = bulk_items + ngroup * 64;
    const int64_t total = g.batch * g.tiles * items_per_tile;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t e = i / (g.tiles * items_per_tile);
        int64_t rem = i - e * g.tiles * items_per_tile;
        int64_t tile = rem / items_per_tile;
        int64_t it = rem - tile * items_per_tile;
        int r = (int)(it & 63);
        int64_t row = tile * 64 + r;
        bool live = row < g.rows;
        uint8_t *packed_base = (direction == 0 ? dst : const_cast<uint8_t *>(src)) +
                               e * g.matrix_bytes + tile * g.tile_bytes;
        const uint8_t *ggml_row = (direction == 0 ? src : dst) + e * g.ggml_matrix_bytes +
                                  row * g.ggml_row_bytes;
        if (it < bulk_items) {
            int64_t bc = it >> 6;                 // b * nchunk + c
            int64_t b = bc / nchunk;
            int c = (int)(bc - b * nchunk);
            uint8_t *p = packed_base + it * 16;
            int64_t goff = b * bpb + lq_chunk_src(t, c);
            if (direction == 0) {
                uint8_t tmp[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) tmp[k] = live ? ggml_row[goff + k] : 0;
                uint4 v;
                __builtin_memcpy(&v, tmp, 16);
                *reinterpret_cast<uint4 *>(p) = v;
            } else if (live) {
                uint4 v = *reinterpret_cast<const uint4 *>(p);
                uint8_t tmp[16];
                __builtin_memcpy(tmp, &v, 16);
                uint8_t *q = const_cast<uint8_t *>(ggml_row) + goff;
#pragma unroll
                for (int k = 0; k < 16; ++k) q[k] = tmp[k];
            }
        } else {
            int64_t gi = (it - bulk_items) >> 6;   // group of 8 blocks
            uint8_t *p = packed_base + g.bulk_bytes + (gi * 64 + r) * 16;
            int dsrc = lq_d16_src(t);
            if (direction == 0) {
                uint8_t tmp[16];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    int64_t b = gi * 8 + k;
                    bool ok = live && b < g.nb;
                    tmp[2 * k] = ok ? ggml_row[b * bpb + dsrc] : 0;
                    tmp[2 * k + 1] = ok ? ggml_row[b * bpb + dsrc + 1] : 0;
                }
                uint4 v;
                __builtin_memcpy(&v, tmp, 16);
                *reinterpret_cast<uint4 *>(p) = v;
            } else if (live) {
                uint4 v = *reinterpret_cast<const uint4 *>(p);
                uint8_t tmp[16];
                __builtin_memcpy(tmp, &v, 16);
                uint8_t *q = const_cast<uint8_t *>(ggml_row);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    int64_t b = gi * 8 + k;
                    if (b < g.nb) {
                        q[b * bpb + dsrc] = tmp[2 * k];
                        q[b * bpb + dsrc + 1] = tmp[2 * k + 1];
                    }
                }
            }
        }
    }
}

int launch_repack(const lq_geom &g, const uint8_t *src, uint8_t *dst, int direction, hipStream_t s) {
    const int64_t ngroup = lq_has_d16(g.type) ? (g.nb + 7) / 8 : 0;
    const int64_t total = g.batch * g.tiles * (g.nb * lq_nchunk(g.type) + ngroup) * 64;
    if (total <= 0) return LOCALAI_OK;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, src, dst, direction);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
