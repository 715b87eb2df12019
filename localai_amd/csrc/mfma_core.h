// mfma_core.h -- building blocks of the decode matvecs on i8 MFMA
// (v_mfma_i32_16x16x64_i8) over the tile form of Q4_K / Q6_K matrices.
//
// Tile form: rows in tiles of 16, and per (tile, super-block) one block whose
// quant bytes are stored so that each 16-byte lane slice is directly the B
// operand of the MFMA (lane l: column n = l % 16, k = 16 (l / 16) .. + 15,
// bytes in k order). Lane L = n + 16c of a block holds row n's bytes
// 8c .. 8c + 7 of two 32-byte quant chunks, so every load instruction of a
// wave reads 1 KiB contiguous.
//   Q4_K block (2304 B): qs piece 0 [64][16 B] (chunks 0, 1), qs piece 1
//     [64][16 B] (chunks 2, 3), headers [16 rows][16 B] (d, dmin, scales)
//   Q6_K block (3360 B): ql piece h [64][16 B] (ql[64h + 8c ..], ql[64h + 32
//     + 8c ..]), qh [64][16 B] (qh[8c ..], qh[32 + 8c ..]), int8 scales
//     [16 rows][16 B], d [16 rows][2 B]
//   Q8_0 block of 8 GGML blocks (4352 B): piece p [64][16 B] (quants 8c ..
//     8c + 7 of blocks 2p and 2p + 1), d [16 rows][8 x 2 B]
//
// Arithmetic, per (tile, super-block):
//   B = the quants as unsigned bytes (Q4_K: a nibble, 0..15, masked in place;
//       Q6_K: low nibble | high 2 bits << 4, 0..63), four MFMAs of 64 values
//   A = x as three int8 pieces per value: with 2^s chosen per scale group so
//       that max |x| 2^s lies in [32, 64),
//         x 2^s = p0 + p1 / 128 + p2 / 16384 + e,  |e| <= 2^-15,
//       each piece rounded with the 1.5 * 2^23 magic-number add (exact steps).
//       A row m = 4 slot + piece carries one scale group in its k range and
//       zero elsewhere (block diagonal), so D[4 slot + piece][n] is the exact
//       integer dot product of that group's quants with one piece.
//   The lane holding D rows 4q .. 4q + 2 of column n then forms
//     sum_group q x = 2^-s (D0 + D1 / 128 + D2 / 16384)
//   and applies the group's scales -- the factorisation of
//   engine/native_quant.cpp:183-231 (Q4_K) and :298-341 (Q6_K) without
//   quantising x (relative error of x about 1e-6 of the group maximum).
//
// x staging: each wave converts the x values of its super-blocks into
// [group][piece][k / 8][8 bytes] in its own LDS region plus per-group
// (sum of x, 2^-s); each lane reads the 8 bytes of its (row, k) slice and
// places them in the low or high half of its A register with an AND mask.
#pragma once
#include "gemv_core.h"

namespace lq {

typedef int mt_i4 __attribute__((ext_vector_type(4)));

constexpr int MT_ROWS = 16;
constexpr int MT_Q4K_BLOCK = 2304;
constexpr int MT_Q6K_BLOCK = 3360;     // ql 2 x 1 KiB, qh 1 KiB, scales 16 x 16 B, d 16 x 2 B
constexpr int MT_Q80_BLOCK = 4352;     // 8 Q8_0 blocks: 4 block-pair pieces x 1 KiB, d 16 rows x 8 x 2 B
constexpr int MT_XBYTES = 1024 + 64;   // Q4_K per super-block: x pieces + 8 x (group sum, 2^-s)
constexpr int MT6_XBYTES = 1024 + 128; // Q6_K per super-block: x pieces + 16 x (sub-block sum, 2^-s)

__host__ __device__ constexpr int mt_block_bytes(int t) {
    return t == LQ_Q4_K ? MT_Q4K_BLOCK : t == LQ_Q6_K ? MT_Q6K_BLOCK : MT_Q80_BLOCK;
}
// 256-value blocks per row in the tile form (Q8_0: eight GGML blocks, the
// last one zero-padded)
__host__ __device__ inline int64_t mt_nsb(const lq_geom &g) { return g.type == LQ_Q8_0 ? (g.nb + 7) / 8 : g.nb; }
__host__ __device__ constexpr int mt_xbytes(int t) { return t == LQ_Q6_K ? MT6_XBYTES : MT_XBYTES; }

// LDS of a workgroup running mt_pass: per-wave x regions, cross-wave partial
// sums, final row sums
__host__ __device__ constexpr size_t mt_lds_bytes(int type, int waves, int spw, int nx, int rt) {
    return (size_t)waves * spw * nx * mt_xbytes(type) + (size_t)waves * rt * 64 * 4 + (size_t)rt * 16 * 4;
}

// Value of lane l ^ 1 (quad_perm [1,0,3,2], 0xB1), l ^ 2 (quad_perm [2,3,0,1],
// 0x4E) or 7 - l inside each 8 (row_half_mirror, 0x141): DPP moves used for
// sums / maxima over aligned groups of 4 or 8 lanes without an LDS round trip.
template <int CTRL>
__device__ __forceinline__ float mt_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

constexpr float MT_MAGIC = 12582912.0f;   // 1.5 * 2^23: x + MAGIC holds rint(x) in its low mantissa bits

// Three int8 pieces of a = x 2^s (|a| < 64) as the low bytes of t0, t1, t2:
// a = p0 + p1 / 128 + p2 / 16384 + e. Every step is exact except the three
// roundings to integers (fma of exactly representable terms, products by
// powers of two, differences of nearby numbers).
__device__ __forceinline__ void mt_split(float x, float S, float S128, uint32_t &b0, uint32_t &b1,
                                         uint32_t &b2) {
    const float t0 = __builtin_fmaf(x, S, MT_MAGIC);
    const float r1 = __builtin_fmaf(x, S128, __builtin_fmaf(-128.0f, t0, 128.0f * MT_MAGIC));
    const float t1 = r1 + MT_MAGIC;
    const float r2 = __builtin_fmaf(r1, 128.0f, __builtin_fmaf(-128.0f, t1, 128.0f * MT_MAGIC));
    const float t2 = r2 + MT_MAGIC;
    b0 = __builtin_bit_cast(uint32_t, t0);
    b1 = __builtin_bit_cast(uint32_t, t1);
    b2 = __builtin_bit_cast(uint32_t, t2);
}

// Low bytes of four words packed into one (byte i from word i). v_perm_b32:
// selector bytes 0..3 pick bytes of the second operand, 4..7 of the first,
// 0x0C gives zero.
__device__ __forceinline__ uint32_t mt_pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);
    const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x0C0C0400u);
    return lo | (hi << 16);
}

// Scale exponent s for a group maximum m: m 2^s in [32, 64); 0 for zero,
// infinite or NaN maxima; clamped so 2^s, 2^(s+7) and 2^-s stay normal.
__device__ __forceinline__ int mt_group_shift(float gmax) {
    int sh = 0;
    if (gmax > 0.0f && gmax <= 3.4e38f) {
        int e;
        frexpf(gmax, &e);
        sh = 6 - e;
        sh = sh > 118 ? 118 : sh < -120 ? -120 : sh;
    }
    return sh;
}

// Convert four x values (natural positions 4 lane .. + 3 of a super-block)
// into pieces and store them; returns (sum, 2^-s) of the lane's group.
template <int GL>   // lanes per scale group: 8 (32 values) or 4 (16 values)
__device__ __forceinline__ float2 mt_stage_x(float4 v, uint8_t *dst, int stride_piece) {
    float gs = (v.x + v.y) + (v.z + v.w);
    float gm = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    gs += mt_dpp<0xB1>(gs);
    gm = fmaxf(gm, mt_dpp<0xB1>(gm));
    gs += mt_dpp<0x4E>(gs);
    gm = fmaxf(gm, mt_dpp<0x4E>(gm));
    if (GL == 8) {
        gs += mt_dpp<0x141>(gs);
        gm = fmaxf(gm, mt_dpp<0x141>(gm));
    }
    const int sh = mt_group_shift(gm);
    const float S = ldexpf(1.0f, sh), S128 = ldexpf(1.0f, sh + 7);
    uint32_t a0, a1, a2, b0, b1, b2, c0, c1, c2, d0, d1, d2;
    mt_split(v.x, S, S128, a0, a1, a2);
    mt_split(v.y, S, S128, b0, b1, b2);
    mt_split(v.z, S, S128, c0, c1, c2);
    mt_split(v.w, S, S128, d0, d1, d2);
    *reinterpret_cast<uint32_t *>(dst) = mt_pack4(a0, b0, c0, d0);
    *reinterpret_cast<uint32_t *>(dst + stride_piece) = mt_pack4(a1, b1, c1, d1);
    *reinterpret_cast<uint32_t *>(dst + 2 * stride_piece) = mt_pack4(a2, b2, c2, d2);
    return make_float2(gs, ldexpf(1.0f, -sh));
}

// A operand: the lane's 8 bytes in the low (mlo) or high (mhi) half, or zero
__device__ __forceinline__ mt_i4 mt_place(uint2 r, uint32_t mlo, uint32_t mhi) {
    return mt_i4{(int)(r.x & mlo), (int)(r.y & mlo), (int)(r.x & mhi), (int)(r.y & mhi)};
}

// sum over the group of q x from D rows (piece 0, 1, 2), before 2^-s
__device__ __forceinline__ float mt_pieces(mt_i4 D) {
    return __builtin_fmaf((float)D[2], 0x1p-14f, __builtin_fmaf((float)D[1], 0x1p-7f, (float)D[0]));
}

__device__ __forceinline__ mt_i4 mt_as_i4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return mt_i4{(int)a, (int)b, (int)c, (int)d};
}

// ------------------------------------------------------- per-type pieces

// Weights of one (tile, super-block) in registers
template <int TYPE> struct MtW;
template <> struct MtW<LQ_Q4_K> { uint4 q0, q1, hd; };
template <> struct MtW<LQ_Q6_K> { uint4 l0, l1, qh, sc; uint32_t d; };
template <> struct MtW<LQ_Q8_0> { uint4 p[4], d; };

template <int TYPE>
__device__ __forceinline__ MtW<TYPE> mt_load_w(const uint8_t *blk, int lane);
template <>
__device__ __forceinline__ MtW<LQ_Q4_K> mt_load_w<LQ_Q4_K>(const uint8_t *blk, int lane) {
    MtW<LQ_Q4_K> w;
    w.q0 = ld16_nt(blk + 16 * lane);
    w.q1 = ld16_nt(blk + 1024 + 16 * lane);
    w.hd = ld16(blk + 2048 + 16 * (lane & 15));
    return w;
}
template <>
__device__ __forceinline__ MtW<LQ_Q8_0> mt_load_w<LQ_Q8_0>(const uint8_t *blk, int lane) {
    MtW<LQ_Q8_0> w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w.p[i] = ld16_nt(blk + 1024 * i + 16 * lane);
    w.d = ld16(blk + 4096 + 16 * (lane & 15));
    return w;
}
template <>
__device__ __forceinline__ MtW<LQ_Q6_K> mt_load_w<LQ_Q6_K>(const uint8_t *blk, int lane) {
    MtW<LQ_Q6_K> w;
    w.l0 = ld16_nt(blk + 16 * lane);
    w.l1 = ld16_nt(blk + 1024 + 16 * lane);
    w.qh = ld16_nt(blk + 2048 + 16 * lane);
    w.sc = ld16(blk + 3072 + 16 * (lane & 15));
    w.d = *reinterpret_cast<const uint16_t *>(blk + 3328 + 2 * (lane & 15));
    return w;
}

// x of one super-block (lane l: values 4l .. 4l + 3) -> the wave's LDS region
//   Q4_K: pieces [group 8][piece 4][k / 8: 4][8 B], then (sum, 2^-s) per group
//   Q6_K: pieces [sub-block 16][piece 4][k / 8: 2][8 B], then per sub-block
template <int TYPE>
__device__ __forceinline__ void mt_stage(float4 v, uint8_t *frag, int lane) {
    if (TYPE == LQ_Q4_K || TYPE == LQ_Q8_0) {   // groups of 32 values (Q8_0: its blocks)
        const int g = lane >> 3;
        const float2 gd = mt_stage_x<8>(v, frag + g * 128 + ((lane & 7) >> 1) * 8 + 4 * (lane & 1), 32);
        if ((lane & 7) == 0) reinterpret_cast<float2 *>(frag + 1024)[g] = gd;
    } else {
        const int j = lane >> 2;
        const float2 gd = mt_stage_x<4>(v, frag + j * 64 + ((lane & 3) >> 1) * 8 + 4 * (lane & 1), 16);
        if ((lane & 3) == 0) reinterpret_cast<float2 *>(frag + 1024)[j] = gd;
    }
}

// Per-lane constants of the A operand and of the D rows.
// Q4_K: MFMA t takes qs piece t / 2, nibble t % 2: bytes 0..7 of lane group q
// are values 8q .. 8q + 7 of group gA(t), bytes 8..15 those of group
// gB(t) = gA(t) + 2, with gA = 0, 1, 4, 5. MFMAs 0, 1 accumulate into D0 and
// 2, 3 into D1; MFMA t uses A slots 2 (t % 2) (group gA) and 2 (t % 2) + 1
// (group gB), so D lane group q ends with group (q / 2) + 2 (q % 2) (+ 4 in D1).
// Q6_K: MFMA i covers values 64 i .. 64 i + 63 (half i / 2, ql nibble i % 2):
// bytes 0..7 of lane group q are sub-block 4i + q / 2, values 8 (q % 2) + 0..7,
// bytes 8..15 sub-block 4i + 2 + q / 2. Each MFMA has its own D; A slot =
// sub-block 4i + slot, so D lane group q holds sub-block 4i + q.
template <int TYPE> struct MtLane;
template <> struct MtLane<LQ_Q4_K> {
    uint32_t lo[4], hi[4];   // A masks per MFMA
    int aoff, gd;
};
template <> struct MtLane<LQ_Q6_K> {
    uint32_t lo, hi;
    int aoff, q;
};
template <> struct MtLane<LQ_Q8_0> {
    uint32_t lo[4], hi[4];   // A masks per MFMA
    int aoff, q;
};

template <int TYPE>
__device__ __forceinline__ MtLane<TYPE> mt_lane(int lane);
template <>
__device__ __forceinline__ MtLane<LQ_Q4_K> mt_lane<LQ_Q4_K>(int lane) {
    MtLane<LQ_Q4_K> L;
    const int m = lane & 15, q = lane >> 4, slot = m >> 2, pc = m & 3;
    const int ga = (slot >> 1) + 2 * (slot & 1);   // group of this lane's A row in MFMAs t = slot / 2, + 2
    const uint32_t on = pc < 3 ? ~0u : 0u;
    const uint32_t mlo = (slot & 1) ? 0u : on, mhi = (slot & 1) ? on : 0u;
    const uint32_t ev = (slot >> 1) ? 0u : ~0u, od = ~ev;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        L.lo[t] = mlo & ((t & 1) ? od : ev);
        L.hi[t] = mhi & ((t & 1) ? od : ev);
    }
    L.aoff = ga * 128 + pc * 32 + q * 8;
    L.gd = (q >> 1) + 2 * (q & 1);
    return L;
}
// Q8_0: MFMA t takes piece t, whose lane group q holds quants 8q .. 8q + 7
// of blocks 2t (bytes 0..7) and 2t + 1 (bytes 8..15). MFMAs 0, 1 accumulate
// into D0 and 2, 3 into D1; MFMA t uses A slots 2 (t % 2) (block 2t, low
// half) and 2 (t % 2) + 1 (block 2t + 1, high half), so A slot s reads block
// s (MFMAs 0, 1) or s + 4 (MFMAs 2, 3), and D lane group q ends with block q
// (D0) and q + 4 (D1).
template <>
__device__ __forceinline__ MtLane<LQ_Q8_0> mt_lane<LQ_Q8_0>(int lane) {
    MtLane<LQ_Q8_0> L;
    const int m = lane & 15, q = lane >> 4, slot = m >> 2, pc = m & 3;
    const uint32_t on = pc < 3 ? ~0u : 0u;
    const uint32_t mlo = (slot & 1) ? 0u : on, mhi = (slot & 1) ? on : 0u;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t act = (t & 1) == (slot >> 1) ? ~0u : 0u;
        L.lo[t] = mlo & act;
        L.hi[t] = mhi & act;
    }
    L.aoff = slot * 128 + pc * 32 + q * 8;
    L.q = q;
    return L;
}
template <>
__device__ __forceinline__ MtLane<LQ_Q6_K> mt_lane<LQ_Q6_K>(int lane) {
    MtLane<LQ_Q6_K> L;
    const int m = lane & 15, q = lane >> 4, slot = m >> 2, pc = m & 3;
    const uint32_t on = (pc < 3 && (slot & 1) == (q >> 1)) ? ~0u : 0u;
    L.lo = (slot >> 1) ? 0u : on;
    L.hi = (slot >> 1) ? on : 0u;
    L.aoff = slot * 64 + pc * 16 + (q & 1) * 8;
    L.q = q;
    return L;
}

// A operands and group data of one staged super-block
template <int TYPE> struct MtA;
template <> struct MtA<LQ_Q4_K> { mt_i4 A[4]; float2 x0, x1; };
template <> struct MtA<LQ_Q6_K> { mt_i4 A[4]; float2 xg[4]; };
template <> struct MtA<LQ_Q8_0> { mt_i4 A[4]; float2 x0, x1; };

template <int TYPE>
__device__ __forceinline__ MtA<TYPE> mt_load_a(const uint8_t *frag, const MtLane<TYPE> &L);
template <>
__device__ __forceinline__ MtA<LQ_Q4_K> mt_load_a<LQ_Q4_K>(const uint8_t *frag, const MtLane<LQ_Q4_K> &L) {
    MtA<LQ_Q4_K> a;
    const uint2 r0 = *reinterpret_cast<const uint2 *>(frag + L.aoff);
    const uint2 r1 = *reinterpret_cast<const uint2 *>(frag + L.aoff + 512);
    a.A[0] = mt_place(r0, L.lo[0], L.hi[0]);
    a.A[1] = mt_place(r0, L.lo[1], L.hi[1]);
    a.A[2] = mt_place(r1, L.lo[2], L.hi[2]);
    a.A[3] = mt_place(r1, L.lo[3], L.hi[3]);
    a.x0 = reinterpret_cast<const float2 *>(frag + 1024)[L.gd];
    a.x1 = reinterpret_cast<const float2 *>(frag + 1024)[L.gd + 4];
    return a;
}
template <>
__device__ __forceinline__ MtA<LQ_Q8_0> mt_load_a<LQ_Q8_0>(const uint8_t *frag, const MtLane<LQ_Q8_0> &L) {
    MtA<LQ_Q8_0> a;
    const uint2 r0 = *reinterpret_cast<const uint2 *>(frag + L.aoff);         // block slot
    const uint2 r1 = *reinterpret_cast<const uint2 *>(frag + L.aoff + 512);   // block slot + 4
    a.A[0] = mt_place(r0, L.lo[0], L.hi[0]);
    a.A[1] = mt_place(r0, L.lo[1], L.hi[1]);
    a.A[2] = mt_place(r1, L.lo[2], L.hi[2]);
    a.A[3] = mt_place(r1, L.lo[3], L.hi[3]);
    a.x0 = reinterpret_cast<const float2 *>(frag + 1024)[L.q];
    a.x1 = reinterpret_cast<const float2 *>(frag + 1024)[L.q + 4];
    return a;
}
template <>
__device__ __forceinline__ MtA<LQ_Q6_K> mt_load_a<LQ_Q6_K>(const uint8_t *frag, const MtLane<LQ_Q6_K> &L) {
    MtA<LQ_Q6_K> a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a.A[i] = mt_place(*reinterpret_cast<const uint2 *>(frag + L.aoff + 256 * i), L.lo, L.hi);
        a.xg[i] = reinterpret_cast<const float2 *>(frag + 1024)[4 * i + L.q];
    }
    return a;
}

// acc + the lane's part of one (tile, super-block) dot product
template <int TYPE>
__device__ __forceinline__ float mt_dot(const MtW<TYPE> &w, const MtA<TYPE> &a, const MtLane<TYPE> &L, float acc);
template <>
__device__ __forceinline__ float mt_dot<LQ_Q4_K>(const MtW<LQ_Q4_K> &w, const MtA<LQ_Q4_K> &a,
                                                 const MtLane<LQ_Q4_K> &L, float acc) {
    const uint4 p = w.q0, r = w.q1;
    const uint32_t M = 0x0F0F0F0Fu;
    mt_i4 D0 = mt_i4{0, 0, 0, 0}, D1 = mt_i4{0, 0, 0, 0};
    D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[0], mt_as_i4(p.x & M, p.y & M, p.z & M, p.w & M), D0, 0, 0, 0);
    D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        a.A[1], mt_as_i4((p.x >> 4) & M, (p.y >> 4) & M, (p.z >> 4) & M, (p.w >> 4) & M), D0, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[2], mt_as_i4(r.x & M, r.y & M, r.z & M, r.w & M), D1, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        a.A[3], mt_as_i4((r.x >> 4) & M, (r.y >> 4) & M, (r.z >> 4) & M, (r.w >> 4) & M), D1, 0, 0, 0);
    // 6-bit scale / min of groups gd (< 4) and gd + 4 (engine/dequant.py:107-113)
    const uint4 h = w.hd;
    const uint32_t s0 = __builtin_amdgcn_ubfe(h.y, 8 * L.gd, 8);
    const uint32_t s4 = __builtin_amdgcn_ubfe(h.z, 8 * L.gd, 8);
    const uint32_t s8 = __builtin_amdgcn_ubfe(h.w, 8 * L.gd, 8);
    const float sc0 = (float)(s0 & 63u), mn0 = (float)(s4 & 63u);
    const float sc1 = (float)((s8 & 15u) | ((s0 >> 6) << 4)), mn1 = (float)((s8 >> 4) | ((s4 >> 6) << 4));
    const float d = f16_to_f32(h.x), dmin = f16_to_f32(h.x >> 16);
    const float v = __builtin_fmaf(sc1 * a.x1.y, mt_pieces(D1), sc0 * a.x0.y * mt_pieces(D0));
    const float u = __builtin_fmaf(mn1, a.x1.x, mn0 * a.x0.x);
    return __builtin_fmaf(-dmin, u, __builtin_fmaf(d, v, acc));
}
template <>
__device__ __forceinline__ float mt_dot<LQ_Q8_0>(const MtW<LQ_Q8_0> &w, const MtA<LQ_Q8_0> &a,
                                                 const MtLane<LQ_Q8_0> &L, float acc) {
    // the int8 quants are the B operand as they are (engine/dequant.py:75-78)
    auto B = [](uint4 v) { return mt_as_i4(v.x, v.y, v.z, v.w); };
    mt_i4 D0 = mt_i4{0, 0, 0, 0}, D1 = mt_i4{0, 0, 0, 0};
    D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[0], B(w.p[0]), D0, 0, 0, 0);
    D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[1], B(w.p[1]), D0, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[2], B(w.p[2]), D1, 0, 0, 0);
    D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[3], B(w.p[3]), D1, 0, 0, 0);
    // d of blocks q and q + 4 of the row (f16 pairs in the header words)
    const uint32_t w0 = (L.q >> 1) ? w.d.y : w.d.x, w1 = (L.q >> 1) ? w.d.w : w.d.z;
    const int sh = 16 * (L.q & 1);
    const float d0 = f16_to_f32(w0 >> sh), d1 = f16_to_f32(w1 >> sh);
    const float v = __builtin_fmaf(d1 * a.x1.y, mt_pieces(D1), d0 * a.x0.y * mt_pieces(D0));
    return acc + v;
}
template <>
__device__ __forceinline__ float mt_dot<LQ_Q6_K>(const MtW<LQ_Q6_K> &w, const MtA<LQ_Q6_K> &a,
                                                 const MtLane<LQ_Q6_K> &L, float acc) {
    // q = (ql >> 4 (i % 2)) & 15 | ((qh >> 2 j) & 3) << 4 (engine/dequant.py:146-165),
    // unsigned; the -32 offset goes through the sub-block sums of x
    const uint32_t K = 0x0F0F0F0Fu;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 l = (i >> 1) ? w.l1 : w.l0;
        const uint32_t e0 = (i >> 1) ? w.qh.z : w.qh.x;
        const uint32_t e1 = (i >> 1) ? w.qh.w : w.qh.y;
        mt_i4 B;
        if (i & 1)
            B = mt_as_i4(((l.x >> 4) & K) | (e0 & 0x30303030u), ((l.y >> 4) & K) | (e1 & 0x30303030u),
                         ((l.z >> 4) & K) | ((e0 >> 2) & 0x30303030u), ((l.w >> 4) & K) | ((e1 >> 2) & 0x30303030u));
        else
            B = mt_as_i4((l.x & K) | ((e0 << 4) & 0x30303030u), (l.y & K) | ((e1 << 4) & 0x30303030u),
                         (l.z & K) | ((e0 << 2) & 0x30303030u), (l.w & K) | ((e1 << 2) & 0x30303030u));
        const mt_i4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.A[i], B, mt_i4{0, 0, 0, 0}, 0, 0, 0);
        const uint32_t sw = i == 0 ? w.sc.x : i == 1 ? w.sc.y : i == 2 ? w.sc.z : w.sc.w;
        const float scf = (float)(int)__builtin_amdgcn_sbfe((int)sw, 8 * L.q, 8);   // the builtin returns unsigned
        s = __builtin_fmaf(scf, __builtin_fmaf(mt_pieces(D), a.xg[i].y, -32.0f * a.xg[i].x), s);
    }
    return __builtin_fmaf(f16_to_f32(w.d), s, acc);
}

// ------------------------------------------------------- workgroup pieces
// Wave w of a workgroup owns super-blocks sb0 = w SPW .. sb0 + nsb - 1 of
// every tile. Loads are unconditional (clamped indices) so that all of them
// are in flight before the first use.

__device__ __forceinline__ int mt_nsb(int nb, int sb0, int spw) {
    const int n = nb - sb0;
    return n < 0 ? 0 : n > spw ? spw : n;
}

// x values of the wave's super-blocks (lane l: 4l .. 4l + 3 of each)
template <int SPW>
__device__ __forceinline__ void mt_load_x(float4 (&xv)[SPW], const float *x, int nb, int sb0, int lane) {
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;
        xv[k] = *reinterpret_cast<const float4 *>(x + 256 * (int64_t)sb + 4 * lane);
    }
}

// weight blocks of the wave's super-blocks of one tile (tile = its block 0)
template <int TYPE, int SPW>
__device__ __forceinline__ void mt_load_tile(MtW<TYPE> (&w)[SPW], const uint8_t *tile, int nb, int sb0, int nsb,
                                             int lane) {
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int kk = k < nsb ? k : 0;
        const int sb = sb0 + kk < nb ? sb0 + kk : nb - 1;
        w[k] = mt_load_w<TYPE>(tile + (int64_t)sb * mt_block_bytes(TYPE), lane);
    }
}

// Dot products of RT tiles with NX x vectors (NX = 1: one x for every tile;
// NX = RT: x[t] for tile t). Returns after a barrier with fin[16 t + n] =
// row n of tile t, summed over the workgroup's waves in a fixed order.
// smem: mt_lds_bytes(TYPE, waves, SPW, NX, RT) bytes.
template <int TYPE, int SPW, int RT, int NX>
__device__ __forceinline__ void mt_pass(const MtW<TYPE> (&w)[RT][SPW], const float4 (&xv)[NX][SPW], int nsb,
                                        uint8_t *smem, float *&fin) {
    constexpr int XB = mt_xbytes(TYPE);
    const int lane = lane_id(), wv = wave_id(), nw = blockDim.x >> 6;
    uint8_t *wl = smem + wv * SPW * NX * XB;
    float *red = reinterpret_cast<float *>(smem + nw * SPW * NX * XB);   // [nw][RT][64]
    fin = red + nw * RT * 64;
#pragma unroll
    for (int j = 0; j < NX; ++j)
#pragma unroll
        for (int k = 0; k < SPW; ++k) mt_stage<TYPE>(xv[j][k], wl + (j * SPW + k) * XB, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    const MtLane<TYPE> L = mt_lane<TYPE>(lane);
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k >= nsb) break;
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const MtA<TYPE> a = mt_load_a<TYPE>(wl + (j * SPW + k) * XB, L);
#pragma unroll
            for (int t = 0; t < RT; ++t)
                if (NX == 1 || t == j) acc[t] = mt_dot<TYPE>(w[t][k], a, L, acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(wv * RT + t) * 64 + lane] = acc[t];
    __syncthreads();
    const int i = threadIdx.x;
    if (i < RT * 16) {
        const int t = i >> 4, n = i & 15;
        float s = 0.0f;
        for (int kk = 0; kk < nw; ++kk) {
            const float *r = red + (kk * RT + t) * 64 + n;
            s += (r[0] + r[16]) + (r[32] + r[48]);
        }
        fin[i] = s;
    }
    __syncthreads();
}

// Software-pipelined form of the per-wave work of mt_pass for one x: the
// wave's super-blocks of RT tiles stream through two register sets, so the
// dot products of block k run while blocks k + 1 and k + 2 are in flight and
// a wave never holds more than two blocks of weights. tile[t]: block 0 of
// tile t; the caller has loaded xv (its x loads go out before the weights),
// and prep(xv, x) makes the x that is multiplied, once the first weight
// blocks are requested (a copy when there is nothing else to do).
// Same arithmetic and summation order as mt_pass (identical results).
struct MtCopyX {
    template <int SPW>
    __device__ void operator()(const float4 (&in)[SPW], float4 (&out)[SPW]) const {
#pragma unroll
        for (int k = 0; k < SPW; ++k) out[k] = in[k];
    }
};
template <int TYPE, int SPW, int RT, typename Prep = MtCopyX>
__device__ __forceinline__ void mt_pass_pipe(const uint8_t *const (&tile)[RT], int nb, int sb0, int nsb,
                                             const float4 (&xv)[SPW], uint8_t *smem, float *&fin,
                                             const Prep &prep = Prep{}) {
    constexpr int XB = mt_xbytes(TYPE);
    const int lane = lane_id(), wv = wave_id(), nw = blockDim.x >> 6;
    uint8_t *wl = smem + wv * SPW * XB;
    float *red = reinterpret_cast<float *>(smem + nw * SPW * XB);   // [nw][RT][64]
    fin = red + nw * RT * 64;
    MtW<TYPE> w[2][RT];
    auto load = [&](MtW<TYPE>(&dst)[RT], int k) {
        const int kk = k < nsb ? k : 0;
        const int sb = sb0 + kk < nb ? sb0 + kk : nb - 1;
#pragma unroll
        for (int t = 0; t < RT; ++t) dst[t] = mt_load_w<TYPE>(tile[t] + (int64_t)sb * mt_block_bytes(TYPE), lane);
    };
    load(w[0], 0);
    if (SPW > 1) load(w[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    float4 xp[SPW];
    prep(xv, xp);
#pragma unroll
    for (int k = 0; k < SPW; ++k) mt_stage<TYPE>(xp[k], wl + k * XB, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const MtLane<TYPE> L = mt_lane<TYPE>(lane);
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k < nsb) {
            const MtA<TYPE> a = mt_load_a<TYPE>(wl + k * XB, L);
#pragma unroll
            for (int t = 0; t < RT; ++t) acc[t] = mt_dot<TYPE>(w[k & 1][t], a, L, acc[t]);
        }
        if (k + 2 < SPW) {
            __builtin_amdgcn_sched_barrier(0);
            load(w[k & 1], k + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(wv * RT + t) * 64 + lane] = acc[t];
    __syncthreads();
    const int i = threadIdx.x;
    if (i < RT * 16) {
        const int t = i >> 4, n = i & 15;
        float s = 0.0f;
        for (int kk = 0; kk < nw; ++kk) {
            const float *r = red + (kk * RT + t) * 64 + n;
            s += (r[0] + r[16]) + (r[32] + r[48]);
        }
        fin[i] = s;
    }
    __syncthreads();
}

}  // namespace lq
