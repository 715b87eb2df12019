// GGML block formats and the device-resident "row planes" layout.
// Shared by host and device code.
//
// GGML formats (bytes per block / values per block), engine/dequant.py:8-11:
//   F32(0) 4/1  F16(1) 2/1  Q4_0(2) 18/32  Q4_1(3) 20/32  Q5_0(6) 22/32
//   Q5_1(7) 24/32  Q8_0(8) 34/32  Q4_K(12) 144/256  Q5_K(13) 176/256
//   Q6_K(14) 210/256
//
// Row-planes layout (what a weight handle holds). A row of K values is cut
// into U = ceil(K / 64) units of 64 values:
//   Q4_K/Q5_K  u = 4*sb + p       group pair p (groups 2p, 2p+1) of super-block sb
//   Q6_K       u = 4*sb + 2*h + m values 128h + 32c + 16m + (0..15), c = 0..3,
//                                 of super-block sb (one 16-byte piece of ql,
//                                 of ql+32 and of qh per unit)
//   Q8_0/Q4_0  u                  blocks 2u and 2u+1 (the second is zero
//                                 padding when the row has an odd block count)
// Each GGML field goes to its own plane, rows one after another. Per-unit
// 16-byte pieces are lane-interleaved: units are taken in chunks of 64 (the
// last chunk holds C = U mod 64 units when that is not zero), and piece j of
// the i-th unit of a chunk sits at 16 * (chunk_start * P + j * C + i) inside
// the row (P pieces per unit), so 64 lanes that each fetch piece j of their
// own unit read 1 KiB contiguous with one load instruction.
//
//   Q4_K : P0 qs, 2 pieces/unit (GGML byte 16+32p+16j)   P1 d,dmin,scales (byte 0, 16 B per sb)
//   Q5_K : P0 qs, 2 pieces/unit (byte 48+32p+16j)        P1 qh, 2 pieces per sb (byte 16+16j),
//          interleaved per chunk of 16 super-blocks      P2 d,dmin,scales (byte 0, 16 B per sb)
//   Q6_K : P0 ql, 2 pieces/unit (byte 64h+16m+32j)       P1 qh, 1 piece/unit (byte 128+32h+16m)
//          P2 scales, 4 B/unit: bytes 192+8h+m+2c, c = 0..3 (the unit's four 16-value scales)
//          P3 d (byte 208, 2 B per sb)
//   Q8_0 : P0 qs, 4 pieces/unit (block 2u+(j>>1), byte 2+16(j&1))
//          P1 d of blocks 2u, 2u+1 (4 B/unit)
//   Q4_0 : P0 qs, 2 pieces/unit (block 2u+j, byte 2)     P1 d of blocks 2u, 2u+1 (4 B/unit)
//
// Every piece is 16-byte aligned (GGML's 210- and 34-byte blocks are only
// 2-byte aligned). The repack is lossless and reversible; GGML bytes remain
// the ABI.
#pragma once
#include <stdint.h>

#define LQ_F32 0
#define LQ_F16 1
#define LQ_Q4_0 2
#define LQ_Q4_1 3
#define LQ_Q5_0 6
#define LQ_Q5_1 7
#define LQ_Q8_0 8
#define LQ_Q4_K 12
#define LQ_Q5_K 13
#define LQ_Q6_K 14

#define LQ_MAX_PLANES 4

#ifdef __HIPCC__
#define LQ_HD __host__ __device__
#else
#define LQ_HD
#endif

// values per block; 0 for unknown types
LQ_HD static inline int lq_block_values(int t) {
    switch (t) {
        case LQ_F32: case LQ_F16: return 1;
        case LQ_Q4_0: case LQ_Q4_1: case LQ_Q5_0: case LQ_Q5_1: case LQ_Q8_0: return 32;
        case LQ_Q4_K: case LQ_Q5_K: case LQ_Q6_K: return 256;
        default: return 0;
    }
}

LQ_HD static inline int lq_block_bytes(int t) {
    switch (t) {
        case LQ_F32: return 4;   case LQ_F16: return 2;
        case LQ_Q4_0: return 18; case LQ_Q4_1: return 20;
        case LQ_Q5_0: return 22; case LQ_Q5_1: return 24;
        case LQ_Q8_0: return 34; case LQ_Q4_K: return 144;
        case LQ_Q5_K: return 176; case LQ_Q6_K: return 210;
        default: return 0;
    }
}

// Types that have a row-planes form and matvec / GEMM kernels.
LQ_HD static inline bool lq_repackable(int t) {
    return t == LQ_Q4_0 || t == LQ_Q8_0 || t == LQ_Q4_K || t == LQ_Q5_K || t == LQ_Q6_K;
}

LQ_HD static inline int lq_nplanes(int t) {
    switch (t) {
        case LQ_Q4_K: return 2; case LQ_Q5_K: return 3; case LQ_Q6_K: return 4;
        case LQ_Q8_0: return 2; case LQ_Q4_0: return 2; default: return 0;
    }
}

// Byte offset, inside a row of a lane-interleaved plane, of 16-byte piece j
// of item i: n items per row, P pieces per item, chunks of CH items.
LQ_HD static inline int64_t lq_ilv(int64_t i, int64_t n, int P, int j, int CH) {
    const int64_t c0 = i - i % CH;
    const int64_t C = n - c0 < CH ? n - c0 : CH;
    return 16 * (c0 * P + j * C + (i - c0));
}

struct lq_geom {
    int type;
    int nplanes;
    int64_t rows, cols, batch;   // batch = experts for a 3-D [E, rows, cols] tensor
    int64_t nb;                  // blocks per row
    int64_t nu;                  // 64-value units per row
    int64_t pitch[LQ_MAX_PLANES];   // bytes per row in each plane
    int64_t plane[LQ_MAX_PLANES];   // byte offset of each plane inside one matrix
    int64_t matrix_bytes;        // per expert matrix (256-byte aligned)
    int64_t ggml_row_bytes;      // GGML bytes per row
    int64_t ggml_matrix_bytes;   // GGML bytes per expert matrix
};

LQ_HD static inline int64_t lq_align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

LQ_HD static inline lq_geom lq_make_geom(int t, int64_t rows, int64_t cols, int64_t batch) {
    lq_geom g;
    g.type = t; g.rows = rows; g.cols = cols; g.batch = batch;
    int bv = lq_block_values(t);
    g.nb = bv ? cols / bv : 0;
    g.nu = (cols + 63) / 64;
    g.nplanes = lq_nplanes(t);
    const int64_t U = g.nu, nb = g.nb;
    int64_t pitch[LQ_MAX_PLANES] = {0, 0, 0, 0};
    switch (t) {
        case LQ_Q4_K: pitch[0] = 32 * U; pitch[1] = 16 * nb; break;
        case LQ_Q5_K: pitch[0] = 32 * U; pitch[1] = 32 * nb; pitch[2] = 16 * nb; break;
        case LQ_Q6_K: pitch[0] = 32 * U; pitch[1] = 16 * U; pitch[2] = 4 * U; pitch[3] = 2 * nb; break;
        case LQ_Q8_0: pitch[0] = 64 * U; pitch[1] = 4 * U; break;
        case LQ_Q4_0: pitch[0] = 32 * U; pitch[1] = 4 * U; break;
        default: break;
    }
    int64_t off = 0;
    for (int p = 0; p < LQ_MAX_PLANES; ++p) {
        g.pitch[p] = pitch[p];
        g.plane[p] = off;
        if (p < g.nplanes) off = lq_align256(off + rows * pitch[p]);
    }
    g.matrix_bytes = off;
    g.ggml_row_bytes = g.nb * lq_block_bytes(t);
    g.ggml_matrix_bytes = g.ggml_row_bytes * rows;
    return g;
}
