// GGML block formats and the device-resident ("lane-interleaved") layout.
// Shared by host and device code.
//
// GGML formats (bytes per block / values per block), engine/dequant.py:8-11:
//   F32(0) 4/1  F16(1) 2/1  Q4_0(2) 18/32  Q4_1(3) 20/32  Q5_0(6) 22/32
//   Q5_1(7) 24/32  Q8_0(8) 34/32  Q4_K(12) 144/256  Q5_K(13) 176/256
//   Q6_K(14) 210/256
//
// Lane-interleaved layout used by the matvec/GEMM kernels. A [rows, cols]
// matrix is cut into row-tiles of 64 rows (rows padded with zero bytes). Each
// GGML block is split into 16-byte "chunks" of bulk data plus an optional
// 2-byte scalar field (the fp16 scale d of Q8_0/Q4_0/Q6_K). Inside a row-tile:
//
//   bulk : [block b][chunk c][row-in-tile 0..63][16 B]        nb * nchunk * 1 KiB
//   d16  : [block/8][row-in-tile 0..63][8 x fp16]             ceil(nb/8) * 1 KiB
//
// so one wave (64 lanes, lane = row) fetches chunk c of block b for 64 rows
// with a single fully coalesced 16 B/lane load, and one more 16 B/lane load
// brings the scales of 8 consecutive blocks. The repack is a byte permutation
// (plus zero padding), lossless and reversible; GGML bytes stay the ABI.
//
// Chunk contents per type (byte ranges refer to the GGML block):
//   Q4_K : c0 = [0,16) d,dmin,scales[12];  c1..c8 = qs [16,144)
//   Q5_K : c0 = [0,16) d,dmin,scales;  c1..c2 = qh [16,48);  c3..c10 = qs [48,176)
//   Q6_K : c0..c7 = ql [0,128);  c8..c11 = qh [128,192);  c12 = scales [192,208);  d16 = [208,210)
//   Q8_0 : c0..c1 = qs [2,34);  d16 = [0,2)
//   Q4_0 : c0 = qs [2,18);  d16 = [0,2)
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

#define LQ_TILE_ROWS 64

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

// Types that have a lane-interleaved (repacked) form and matvec/GEMM kernels.
LQ_HD static inline bool lq_repackable(int t) {
    return t == LQ_Q4_0 || t == LQ_Q8_0 || t == LQ_Q4_K || t == LQ_Q5_K || t == LQ_Q6_K;
}

LQ_HD static inline int lq_nchunk(int t) {
    switch (t) {
        case LQ_Q4_K: return 9; case LQ_Q5_K: return 11; case LQ_Q6_K: return 13;
        case LQ_Q8_0: return 2; case LQ_Q4_0: return 1; default: return 0;
    }
}

LQ_HD static inline bool lq_has_d16(int t) {
    return t == LQ_Q6_K || t == LQ_Q8_0 || t == LQ_Q4_0;
}

// GGML byte offset of chunk c inside a block
LQ_HD static inline int lq_chunk_src(int t, int c) {
    switch (t) {
        case LQ_Q6_K: return 16 * c;          // ql, qh, scales are contiguous from 0
        case LQ_Q8_0: return 2 + 16 * c;
        case LQ_Q4_0: return 2;
        default: return 16 * c;               // Q4_K / Q5_K: whole block is chunked
    }
}

LQ_HD static inline int lq_d16_src(int t) { return t == LQ_Q6_K ? 208 : 0; }

struct lq_geom {
    int type;
    int64_t rows, cols, batch;   // batch = experts for a 3-D [E, rows, cols] tensor
    int64_t nb;                  // blocks per row
    int64_t tiles;               // row-tiles per matrix
    int64_t bulk_bytes;          // per tile
    int64_t tile_bytes;          // per tile (bulk + d16)
    int64_t matrix_bytes;        // per expert matrix (tiles * tile_bytes)
    int64_t ggml_row_bytes;      // GGML bytes per row
    int64_t ggml_matrix_bytes;   // GGML bytes per expert matrix
};

LQ_HD static inline lq_geom lq_make_geom(int t, int64_t rows, int64_t cols, int64_t batch) {
    lq_geom g;
    g.type = t; g.rows = rows; g.cols = cols; g.batch = batch;
    int bv = lq_block_values(t);
    g.nb = bv ? cols / bv : 0;
    g.tiles = (rows + LQ_TILE_ROWS - 1) / LQ_TILE_ROWS;
    g.bulk_bytes = g.nb * lq_nchunk(t) * 1024;
    g.tile_bytes = g.bulk_bytes + (lq_has_d16(t) ? ((g.nb + 7) / 8) * 1024 : 0);
    g.matrix_bytes = g.tiles * g.tile_bytes;
    g.ggml_row_bytes = g.nb * lq_block_bytes(t);
    g.ggml_matrix_bytes = g.ggml_row_bytes * rows;
    return g;
}
