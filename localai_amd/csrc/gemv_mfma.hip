// Decode matvec on MFMA for Q4_K and Q6_K: y[r] = sum_c W[r, c] * x[c].
//
// Weights come from a second device form of the matrix, the "tile form": rows
// in tiles of 16, and per (tile, super-block) one block whose quant bytes are
// stored so that each 16-byte lane slice is directly the B operand of
// v_mfma_i32_16x16x64_i8 (lane l: column n = l % 16, k = 16 (l / 16) .. + 15,
// bytes in k order). Lane L = n + 16c of a block holds row n's bytes
// 8c .. 8c + 7 of two 32-byte quant chunks, so every load instruction of a
// wave reads 1 KiB contiguous.
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
#include "gemv_core.h"
#include "internal.h"

namespace lq {

typedef int mt_i4 __attribute__((ext_vector_type(4)));

constexpr int MT_ROWS = 16;
constexpr int MT_MAX_JOBS = 8;        // matrices per fused launch (localai_hip_matvec_many)
constexpr int MT_Q4K_BLOCK = 2304;
constexpr int MT_Q6K_BLOCK = 3360;     // ql 2 x 1 KiB, qh 1 KiB, scales 16 x 16 B, d 16 x 2 B
constexpr int MT_XBYTES = 1024 + 64;   // Q4_K per super-block: x pieces + 8 x (group sum, 2^-s)
constexpr int MT6_XBYTES = 1024 + 128; // Q6_K per super-block: x pieces + 16 x (sub-block sum, 2^-s)

__host__ __device__ constexpr int mt_block_bytes(int t) { return t == LQ_Q4_K ? MT_Q4K_BLOCK : MT_Q6K_BLOCK; }

// 0 when the matrix gets no tile form (other types, or K beyond the 72
// super-blocks the launch plan covers): its matvecs then run on gemv.hip.
int64_t mt_matrix_bytes(const lq_geom &g) {
    if ((g.type != LQ_Q4_K && g.type != LQ_Q6_K) || g.nb > 72) return 0;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    return lq_align256(tiles * g.nb * mt_block_bytes(g.type));
}

// GGML -> tile form, one thread per (matrix, row, super-block). Rows past
// the end of the last tile stay zero (the caller clears the buffer).
__global__ void mt_repack_q4k(lq_geom g, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int64_t dst_matrix_bytes) {
    const int64_t total = g.batch * g.rows * g.nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * g.nb);
        const int64_t rem = i - e * g.rows * g.nb;
        const int64_t row = rem / g.nb, sb = rem - row * g.nb;
        const uint8_t *s = src + e * g.ggml_matrix_bytes + row * g.ggml_row_bytes + sb * 144;
        uint8_t *blk = dst + e * dst_matrix_bytes + ((row / MT_ROWS) * g.nb + sb) * MT_Q4K_BLOCK;
        const int n = (int)(row % MT_ROWS);
        for (int c = 0; c < 4; ++c) {
            const int L = n + 16 * c;
            for (int p = 0; p < 4; ++p)
                for (int b = 0; b < 8; ++b)
                    blk[(p >> 1) * 1024 + L * 16 + (p & 1) * 8 + b] = s[16 + 32 * p + 8 * c + b];
        }
        for (int b = 0; b < 16; ++b) blk[2048 + n * 16 + b] = s[b];
    }
}

// Q6_K tile block, lane L = n + 16c:
//   ql piece h (h = 0, 1) [64][16 B]: ql[64h + 8c ..+7], ql[64h + 32 + 8c ..+7]
//   qh piece [64][16 B]:             qh[8c ..+7],       qh[32 + 8c ..+7]
//   scales [16 rows][16 B] (int8), d [16 rows][2 B]
__global__ void mt_repack_q6k(lq_geom g, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                              int64_t dst_matrix_bytes) {
    const int64_t total = g.batch * g.rows * g.nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / (g.rows * g.nb);
        const int64_t rem = i - e * g.rows * g.nb;
        const int64_t row = rem / g.nb, sb = rem - row * g.nb;
        const uint8_t *s = src + e * g.ggml_matrix_bytes + row * g.ggml_row_bytes + sb * 210;
        uint8_t *blk = dst + e * dst_matrix_bytes + ((row / MT_ROWS) * g.nb + sb) * MT_Q6K_BLOCK;
        const int n = (int)(row % MT_ROWS);
        for (int c = 0; c < 4; ++c) {
            const int L = n + 16 * c;
            for (int h = 0; h < 2; ++h)
                for (int b = 0; b < 8; ++b) {
                    blk[h * 1024 + L * 16 + b] = s[64 * h + 8 * c + b];
                    blk[h * 1024 + L * 16 + 8 + b] = s[64 * h + 32 + 8 * c + b];
                    blk[2048 + L * 16 + 8 * h + b] = s[128 + 32 * h + 8 * c + b];
                }
        }
        for (int b = 0; b < 16; ++b) blk[3072 + n * 16 + b] = s[192 + b];
        blk[3328 + 2 * n] = s[208];
        blk[3328 + 2 * n + 1] = s[209];
    }
}

int launch_mt_repack(const lq_geom &g, const uint8_t *ggml, uint8_t *dst, int64_t dst_matrix_bytes,
                     hipStream_t s) {
    const int64_t total = g.batch * g.rows * g.nb;
    LQ_HIP(hipMemsetAsync(dst, 0, (size_t)(dst_matrix_bytes * g.batch), s));
    if (total <= 0) return LOCALAI_OK;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (g.type == LQ_Q6_K)
        hipLaunchKernelGGL(mt_repack_q6k, dim3((unsigned)blocks), dim3(256), 0, s, g, ggml, dst, dst_matrix_bytes);
    else
        hipLaunchKernelGGL(mt_repack_q4k, dim3((unsigned)blocks), dim3(256), 0, s, g, ggml, dst, dst_matrix_bytes);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
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

// Shared loads of both kernels: x of the wave's super-blocks, then the tile
// blocks. Every load is unconditional (clamped indices) so they all issue
// before the first use.
#define MT_PROLOGUE(XBYTES)                                                                   \
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];                            \
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;                          \
    const int sb0 = w * SPW;                                                                  \
    int nsb = nb - sb0;                                                                       \
    nsb = nsb < 0 ? 0 : nsb > SPW ? SPW : nsb;                                                \
    uint8_t *wl = smem + w * SPW * (XBYTES);                                                  \
    float *red = reinterpret_cast<float *>(smem + nw * SPW * (XBYTES));                       \
    const int64_t tile0 = blk * RT;                                                           \
    float4 xv[SPW];                                                                           \
    _Pragma("unroll") for (int k = 0; k < SPW; ++k) {                                         \
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;                                       \
        xv[k] = *reinterpret_cast<const float4 *>(x + 256 * (int64_t)sb + 4 * lane);          \
    }

// Cross-wave and cross-lane-group sum of acc[RT] into y
#define MT_EPILOGUE                                                                           \
    _Pragma("unroll") for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];   \
    __syncthreads();                                                                          \
    const int i = threadIdx.x;                                                                \
    if (i < RT * 16) {                                                                        \
        const int t = i >> 4, n = i & 15;                                                     \
        float s = 0.0f;                                                                       \
        for (int k = 0; k < nw; ++k) {                                                        \
            const float *r = red + (k * RT + t) * 64 + n;                                     \
            s += (r[0] + r[16]) + (r[32] + r[48]);                                            \
        }                                                                                     \
        const int64_t row = (tile0 + t) * MT_ROWS + n;                                        \
        if (tile0 + t < tiles && row < rows) y[row] = s;                                      \
    }

// ------------------------------------------------------------------- Q4_K
// MFMA t of a super-block takes qs piece t / 2, nibble t % 2: bytes 0..7 of
// lane group q are values 8q .. 8q + 7 of group gA(t), bytes 8..15 those of
// group gB(t) = gA(t) + 2, with gA = 0, 1, 4, 5. MFMAs 0, 1 accumulate into D0
// and 2, 3 into D1; MFMA t uses A slots 2 (t % 2) (group gA) and
// 2 (t % 2) + 1 (group gB), so D lane group q ends with group
// (q / 2) + 2 (q % 2) (+ 4 for D1).
// LDS per super-block: pieces [group 8][piece 4][k / 8: 4][8 B] (1 KiB), then
// (sum, 2^-s) per group.
template <int SPW, int RT>
__device__ __forceinline__ void mt_body_q4k(const uint8_t *__restrict__ Wt, int64_t rows, int nb, int64_t tiles,
                                            const float *__restrict__ x, float *__restrict__ y, int64_t blk) {
    MT_PROLOGUE(MT_XBYTES)
    uint4 q0[RT][SPW], q1[RT][SPW], hd[RT][SPW];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t tile = tile0 + t < tiles ? tile0 + t : tiles - 1;
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            const int kk = k < nsb ? k : 0;
            const int sb = sb0 + kk < nb ? sb0 + kk : nb - 1;
            const uint8_t *blk = Wt + (tile * nb + sb) * MT_Q4K_BLOCK;
            q0[t][k] = ld16(blk + 16 * lane);
            q1[t][k] = ld16(blk + 1024 + 16 * lane);
            hd[t][k] = ld16(blk + 2048 + 16 * (lane & 15));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    {   // lane l: values 4l .. 4l + 3 = group l / 8, k / 8 = (l % 8) / 2, byte 4 (l % 2)
        const int g = lane >> 3;
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            uint8_t *frag = wl + k * MT_XBYTES;
            const float2 gd = mt_stage_x<8>(xv[k], frag + g * 128 + ((lane & 7) >> 1) * 8 + 4 * (lane & 1), 32);
            if ((lane & 7) == 0) reinterpret_cast<float2 *>(frag + 1024)[g] = gd;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    const int m = lane & 15, q = lane >> 4, slot = m >> 2, pc = m & 3;
    const int ga = (slot >> 1) + 2 * (slot & 1);   // A: group of this lane's row in MFMAs t = slot / 2, + 2
    const int gd = (q >> 1) + 2 * (q & 1);         // D: group of this lane's rows in D0 (D1: + 4)
    const uint32_t on = pc < 3 ? ~0u : 0u;
    const uint32_t mlo = (slot & 1) ? 0u : on, mhi = (slot & 1) ? on : 0u;
    const uint32_t ev = (slot >> 1) ? 0u : ~0u, od = ~ev;
    const int aoff = ga * 128 + pc * 32 + q * 8;
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k >= nsb) break;
        const uint8_t *frag = wl + k * MT_XBYTES;
        const uint2 r0 = *reinterpret_cast<const uint2 *>(frag + aoff);
        const uint2 r1 = *reinterpret_cast<const uint2 *>(frag + aoff + 512);
        const mt_i4 A0 = mt_place(r0, mlo & ev, mhi & ev), A1 = mt_place(r0, mlo & od, mhi & od);
        const mt_i4 A2 = mt_place(r1, mlo & ev, mhi & ev), A3 = mt_place(r1, mlo & od, mhi & od);
        const float2 x0 = reinterpret_cast<const float2 *>(frag + 1024)[gd];
        const float2 x1 = reinterpret_cast<const float2 *>(frag + 1024)[gd + 4];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint4 a = q0[t][k], b = q1[t][k];
            const uint32_t M = 0x0F0F0F0Fu;
            mt_i4 D0 = mt_i4{0, 0, 0, 0}, D1 = mt_i4{0, 0, 0, 0};
            D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, mt_as_i4(a.x & M, a.y & M, a.z & M, a.w & M), D0, 0, 0, 0);
            D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                A1, mt_as_i4((a.x >> 4) & M, (a.y >> 4) & M, (a.z >> 4) & M, (a.w >> 4) & M), D0, 0, 0, 0);
            D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, mt_as_i4(b.x & M, b.y & M, b.z & M, b.w & M), D1, 0, 0, 0);
            D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                A3, mt_as_i4((b.x >> 4) & M, (b.y >> 4) & M, (b.z >> 4) & M, (b.w >> 4) & M), D1, 0, 0, 0);
            // 6-bit scale / min of groups gd (< 4) and gd + 4 (engine/dequant.py:107-113)
            const uint4 h = hd[t][k];
            const uint32_t s0 = __builtin_amdgcn_ubfe(h.y, 8 * gd, 8);
            const uint32_t s4 = __builtin_amdgcn_ubfe(h.z, 8 * gd, 8);
            const uint32_t s8 = __builtin_amdgcn_ubfe(h.w, 8 * gd, 8);
            const float sc0 = (float)(s0 & 63u), mn0 = (float)(s4 & 63u);
            const float sc1 = (float)((s8 & 15u) | ((s0 >> 6) << 4)), mn1 = (float)((s8 >> 4) | ((s4 >> 6) << 4));
            const float d = f16_to_f32(h.x), dmin = f16_to_f32(h.x >> 16);
            const float v = __builtin_fmaf(sc1 * x1.y, mt_pieces(D1), sc0 * x0.y * mt_pieces(D0));
            const float u = __builtin_fmaf(mn1, x1.x, mn0 * x0.x);
            acc[t] = __builtin_fmaf(-dmin, u, __builtin_fmaf(d, v, acc[t]));
        }
    }
    MT_EPILOGUE
}

// ------------------------------------------------------------------- Q6_K
// MFMA i of a super-block covers values 64 i .. 64 i + 63 (half i / 2, ql
// nibble i % 2): bytes 0..7 of lane group q are sub-block 4i + q / 2, values
// 8 (q % 2) + 0..7, and bytes 8..15 sub-block 4i + 2 + q / 2. Quants are
// q = (ql >> 4 (i % 2)) & 15 | ((qh >> 2 j) & 3) << 4 (engine/dequant.py:146-165),
// unsigned; the -32 offset goes through the sub-block sums of x. Each MFMA
// has its own D; A slot = sub-block 4i + slot, so D lane group q holds
// sub-block 4i + q.
// LDS per super-block: pieces [sub-block 16][piece 4][k / 8: 2][8 B] (1 KiB),
// then (sum, 2^-s) per sub-block.
template <int SPW, int RT>
__device__ __forceinline__ void mt_body_q6k(const uint8_t *__restrict__ Wt, int64_t rows, int nb, int64_t tiles,
                                            const float *__restrict__ x, float *__restrict__ y, int64_t blk) {
    MT_PROLOGUE(MT6_XBYTES)
    uint4 ql0[RT][SPW], ql1[RT][SPW], qh[RT][SPW], sc[RT][SPW];
    uint32_t dd[RT][SPW];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int64_t tile = tile0 + t < tiles ? tile0 + t : tiles - 1;
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            const int kk = k < nsb ? k : 0;
            const int sb = sb0 + kk < nb ? sb0 + kk : nb - 1;
            const uint8_t *blk = Wt + (tile * nb + sb) * MT_Q6K_BLOCK;
            ql0[t][k] = ld16(blk + 16 * lane);
            ql1[t][k] = ld16(blk + 1024 + 16 * lane);
            qh[t][k] = ld16(blk + 2048 + 16 * lane);
            sc[t][k] = ld16(blk + 3072 + 16 * (lane & 15));
            dd[t][k] = *reinterpret_cast<const uint16_t *>(blk + 3328 + 2 * (lane & 15));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    {   // lane l: values 4l .. 4l + 3 = sub-block l / 4, k / 8 = (l % 4) / 2, byte 4 (l % 2)
        const int j = lane >> 2;
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            uint8_t *frag = wl + k * MT6_XBYTES;
            const float2 gd = mt_stage_x<4>(xv[k], frag + j * 64 + ((lane & 3) >> 1) * 8 + 4 * (lane & 1), 16);
            if ((lane & 3) == 0) reinterpret_cast<float2 *>(frag + 1024)[j] = gd;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    const int m = lane & 15, q = lane >> 4, slot = m >> 2, pc = m & 3;
    const uint32_t on = (pc < 3 && (slot & 1) == (q >> 1)) ? ~0u : 0u;
    const uint32_t mlo = (slot >> 1) ? 0u : on, mhi = (slot >> 1) ? on : 0u;
    const int aoff = slot * 64 + pc * 16 + (q & 1) * 8;
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k >= nsb) break;
        const uint8_t *frag = wl + k * MT6_XBYTES;
        mt_i4 A[4];
        float2 xg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            A[i] = mt_place(*reinterpret_cast<const uint2 *>(frag + aoff + 256 * i), mlo, mhi);
            xg[i] = reinterpret_cast<const float2 *>(frag + 1024)[4 * i + q];
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t L = 0x0F0F0F0Fu;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 l = (i >> 1) ? ql1[t][k] : ql0[t][k];
                const uint32_t e0 = (i >> 1) ? qh[t][k].z : qh[t][k].x;
                const uint32_t e1 = (i >> 1) ? qh[t][k].w : qh[t][k].y;
                mt_i4 B;
                if (i & 1)
                    B = mt_as_i4(((l.x >> 4) & L) | (e0 & 0x30303030u), ((l.y >> 4) & L) | (e1 & 0x30303030u),
                                 ((l.z >> 4) & L) | ((e0 >> 2) & 0x30303030u),
                                 ((l.w >> 4) & L) | ((e1 >> 2) & 0x30303030u));
                else
                    B = mt_as_i4((l.x & L) | ((e0 << 4) & 0x30303030u), (l.y & L) | ((e1 << 4) & 0x30303030u),
                                 (l.z & L) | ((e0 << 2) & 0x30303030u), (l.w & L) | ((e1 << 2) & 0x30303030u));
                const mt_i4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], B, mt_i4{0, 0, 0, 0}, 0, 0, 0);
                const uint32_t sw = i == 0 ? sc[t][k].x : i == 1 ? sc[t][k].y : i == 2 ? sc[t][k].z : sc[t][k].w;
                const float scf = (float)(int)__builtin_amdgcn_sbfe((int)sw, 8 * q, 8);   // the builtin returns unsigned
                s = __builtin_fmaf(scf, __builtin_fmaf(mt_pieces(D), xg[i].y, -32.0f * xg[i].x), s);
            }
            acc[t] = __builtin_fmaf(f16_to_f32(dd[t][k]), s, acc[t]);
        }
    }
    MT_EPILOGUE
}

#undef MT_PROLOGUE
#undef MT_EPILOGUE

// One matrix: workgroup b takes row tiles b RT .. b RT + RT - 1.
template <int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_q4k(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                      int64_t tiles, const float *__restrict__ x,
                                                      float *__restrict__ y) {
    mt_body_q4k<SPW, RT>(Wt, rows, nb, tiles, x, y, blockIdx.x);
}
template <int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_q6k(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                      int64_t tiles, const float *__restrict__ x,
                                                      float *__restrict__ y) {
    mt_body_q6k<SPW, RT>(Wt, rows, nb, tiles, x, y, blockIdx.x);
}

// Several matrices with the same K and the same x in one launch: job j owns
// workgroups blk0[j] .. blk0[j + 1] - 1 (uniform branch per workgroup).
struct MtJobs {
    const uint8_t *Wt[MT_MAX_JOBS];
    float *y[MT_MAX_JOBS];
    int64_t rows[MT_MAX_JOBS];
    int64_t blk0[MT_MAX_JOBS + 1];
    int type[MT_MAX_JOBS];
    int n;
};
template <int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_many(MtJobs jobs, int nb, const float *__restrict__ x) {
    const int64_t b = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < MT_MAX_JOBS; ++i)
        if (i < jobs.n && b >= jobs.blk0[i]) j = i;
    const int64_t tiles = (jobs.rows[j] + MT_ROWS - 1) / MT_ROWS;
    if (jobs.type[j] == LQ_Q6_K) mt_body_q6k<SPW, RT>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j], b - jobs.blk0[j]);
    else mt_body_q4k<SPW, RT>(jobs.Wt[j], jobs.rows[j], nb, tiles, x, jobs.y[j], b - jobs.blk0[j]);
}

// Launch plan: the waves of a workgroup split the super-blocks of one row
// tile (or RT tiles), SPW super-blocks per wave.
//   nb <= 32, >= 768 tiles: SPW = ceil(nb / 16), up to 16 waves, two tiles
//             per workgroup when SPW = 1 (x staged once for both)
//   nb <= 32, fewer tiles:  SPW = ceil(nb / 8), up to 8 waves, one tile per
//             workgroup, so that small matrices still spread over the CUs
//   nb > 32:  SPW = ceil(nb / 12), up to 12 waves (768 threads, so each wave
//             may hold all of its SPW blocks in registers)
struct MtPlan {
    int spw, waves, rt;
};
static MtPlan mt_plan(int nb, int64_t tiles) {
    MtPlan p;
    const bool big = tiles >= 768;
    p.spw = nb > 32 ? (nb + 11) / 12 : big ? (nb + 15) / 16 : (nb + 7) / 8;
    p.waves = (nb + p.spw - 1) / p.spw;
    p.rt = (big && p.spw == 1) ? 2 : 1;
    return p;
}

#define MT_DISPATCH(L)                                         \
    switch (p.spw) {                                           \
        case 1: if (p.rt == 2) L(1, 2, 1024); else L(1, 1, 1024); break; \
        case 2: L(2, 1, 1024); break;                          \
        case 3: L(3, 1, 768); break;                           \
        case 4: L(4, 1, 768); break;                           \
        case 5: L(5, 1, 768); break;                           \
        default: L(6, 1, 768); break;                          \
    }

int launch_matvec_mfma(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, hipStream_t s) {
    if (g.type != LQ_Q4_K && g.type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g.nb;
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    const bool q6 = g.type == LQ_Q6_K;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    const MtPlan p = mt_plan(nb, tiles);
    dim3 grid((unsigned)((tiles + p.rt - 1) / p.rt)), block(64 * p.waves);
    const size_t lds = (size_t)p.waves * p.spw * (q6 ? MT6_XBYTES : MT_XBYTES) + (size_t)p.waves * p.rt * 64 * 4;
#define MT_L(S, R, M)                                                                                     \
    do {                                                                                                  \
        if (q6) hipLaunchKernelGGL((gemv_mfma_q6k<S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y); \
        else hipLaunchKernelGGL((gemv_mfma_q4k<S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y);    \
    } while (0)
    MT_DISPATCH(MT_L)
#undef MT_L
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

int launch_matvec_mfma_many(int n, const lq_geom *const *g, const uint8_t *const *Wt, const float *x,
                            float *const *y, hipStream_t s) {
    if (n < 1 || n > MT_MAX_JOBS) return fail(LOCALAI_EARG, "mfma matvec: 1..8 matrices per fused launch");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g[0]->nb;
    if (nb > 72) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 18432 values)");
    int64_t total_tiles = 0;
    bool any_q6 = false;
    for (int j = 0; j < n; ++j) {
        if (g[j]->type != LQ_Q4_K && g[j]->type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
        if (g[j]->nb != nb) return fail(LOCALAI_EARG, "mfma matvec: fused matrices need the same cols");
        total_tiles += (g[j]->rows + MT_ROWS - 1) / MT_ROWS;
        any_q6 |= g[j]->type == LQ_Q6_K;
    }
    const MtPlan p = mt_plan(nb, total_tiles);
    MtJobs jobs = {};
    jobs.n = n;
    int64_t b = 0;
    for (int j = 0; j < n; ++j) {
        jobs.Wt[j] = Wt[j];
        jobs.y[j] = y[j];
        jobs.rows[j] = g[j]->rows;
        jobs.type[j] = g[j]->type;
        jobs.blk0[j] = b;
        b += ((g[j]->rows + MT_ROWS - 1) / MT_ROWS + p.rt - 1) / p.rt;
    }
    for (int j = n; j <= MT_MAX_JOBS; ++j) jobs.blk0[j] = b;
    dim3 grid((unsigned)b), block(64 * p.waves);
    const size_t lds = (size_t)p.waves * p.spw * (any_q6 ? MT6_XBYTES : MT_XBYTES) + (size_t)p.waves * p.rt * 64 * 4;
#define MT_L(S, R, M) hipLaunchKernelGGL((gemv_mfma_many<S, R, M>), grid, block, lds, s, jobs, nb, x)
    MT_DISPATCH(MT_L)
#undef MT_L
#undef MT_DISPATCH
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
