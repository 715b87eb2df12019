// Decode matvec on MFMA for Q4_K and Q6_K: y[r] = sum_c W[r, c] * x[c].
//
// Weights come from a second device form of the matrix, the "tile form": rows
// in tiles of 16, and per (tile, super-block) one 2304-byte block
//   qs piece 0 [64 lanes][16 B]   qs piece 1 [64 lanes][16 B]   headers [16 rows][16 B]
// where lane L = n + 16c (row n of the tile, 8-value chunk c) holds bytes
// 32p + 8c .. 32p + 8c + 7 of the row's qs for group pairs p = 0, 1 (piece 0)
// and p = 2, 3 (piece 1). That is exactly the B operand of
// v_mfma_f32_16x16x32_f16 (lane l: k = 8 (l / 16) .. + 7, n = l % 16), so
// every load instruction of a wave reads 1 KiB contiguous.
//
// Arithmetic, per (tile, super-block), one MFMA per 32-value group g:
//   B = the group's 4-bit quants as f16 subnormals (bits = q, value q * 2^-24:
//       exact; high nibbles are taken in place, value 16 q * 2^-24)
//   A = x of the group as an exact two-term f16 expansion: x * 2^s = hi + lo
//       (hi = f16(x 2^s), lo = f16(x 2^s - hi); 22 significant bits), in the
//       rows m = 2g (hi) and 2g + 1 (lo) of the 16-row A operand, zero
//       elsewhere (block diagonal)
//   D[m][n] accumulates, after the 8 groups, sum_k q * x_split for every
//   (group, split) in its own row m: products are exact in fp32 and the sums
//   are fp32, so D carries the group dot products at fp32 accuracy.
// Lane l then holds D rows 4 (l / 16) .. + 3 of row n = l % 16: groups 2q
// and 2q + 1 (q = l / 16), both splits, and applies the group scales once:
//   acc += d sc_2q (D0 + D1) + d sc_2q+1 (D2 + D3) / 16   (times 2^24 2^-s)
//        - dmin (mn_2q X_2q + mn_2q+1 X_2q+1)               (X = group sums of x)
// -- the factorisation of engine/native_quant.cpp:183-231 without quantising x.
//
// x staging: each wave converts the x values of its super-blocks into the
// A fragment layout in its own LDS region ([m][c][8 halves] per super-block)
// plus the eight group sums; lane l reads the fragment of its (m, c) into
// A register a[m / 2] with an exec mask, so the other seven A registers of
// the lane stay zero and no VALU work goes into the block-diagonal zeros.
#include "gemv_core.h"
#include "internal.h"

namespace lq {

typedef _Float16 mt_h8 __attribute__((ext_vector_type(8)));
typedef float mt_f4 __attribute__((ext_vector_type(4)));

constexpr int MT_ROWS = 16;
constexpr int MT_Q4K_BLOCK = 2304;
constexpr int MT_Q6K_BLOCK = 3360;     // ql 2 x 1 KiB, qh 1 KiB, scales 16 x 16 B, d 16 x 2 B
constexpr int MT_XBYTES = 1024 + 64;   // Q4_K per super-block: A fragments + 8 x (group sum, scale)
constexpr int MT6_XBYTES = 1024 + 128; // Q6_K per super-block: A fragments + 16 x (sub-block sum, scale)

__host__ __device__ constexpr int mt_block_bytes(int t) { return t == LQ_Q4_K ? MT_Q4K_BLOCK : MT_Q6K_BLOCK; }

int64_t mt_matrix_bytes(const lq_geom &g) {
    if (g.type != LQ_Q4_K && g.type != LQ_Q6_K) return 0;
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

// f16 pairs (bits = byte value) of bytes 0,1 and 2,3 of a masked dword:
// v_perm_b32 selector bytes 0..3 pick bytes of the second operand, 0x0C a zero
__device__ __forceinline__ uint32_t mt_lo_pair(uint32_t m) { return __builtin_amdgcn_perm(0u, m, 0x0C010C00u); }
__device__ __forceinline__ uint32_t mt_hi_pair(uint32_t m) { return __builtin_amdgcn_perm(0u, m, 0x0C030C02u); }
// A fragment of a lane in one MFMA: its x values where the lane's row is
// nonzero, zero elsewhere (mask all ones or all zeros)
__device__ __forceinline__ mt_h8 mt_masked(uint4 f, uint32_t mask) {
    return __builtin_bit_cast(mt_h8, make_uint4(f.x & mask, f.y & mask, f.z & mask, f.w & mask));
}

// B operand of group g (pair g / 2, nibble g % 2) from the lane's two qs pieces
__device__ __forceinline__ mt_h8 mt_b_q4k(uint4 p0, uint4 p1, int g) {
    const uint4 pc = (g >> 2) ? p1 : p0;
    const uint32_t d0 = (g & 2) ? pc.z : pc.x, d1 = (g & 2) ? pc.w : pc.y;
    const uint32_t mask = (g & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const uint32_t m0 = d0 & mask, m1 = d1 & mask;
    uint4 r;
    r.x = mt_lo_pair(m0);
    r.y = mt_hi_pair(m0);
    r.z = mt_lo_pair(m1);
    r.w = mt_hi_pair(m1);
    return __builtin_bit_cast(mt_h8, r);
}

// Sum / max of a value over each aligned group of 8 lanes, in every lane of
// the group: DPP quad_perm [1,0,3,2], quad_perm [2,3,0,1], then
// row_half_mirror (lane i <-> 7 - i inside each 8) -- no LDS round trip.
template <int CTRL>
__device__ __forceinline__ float mt_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float mt_group8_sum(float v) {
    v += mt_dpp<0xB1>(v);
    v += mt_dpp<0x4E>(v);
    return v + mt_dpp<0x141>(v);
}
__device__ __forceinline__ float mt_group8_max(float v) {
    v = fmaxf(v, mt_dpp<0xB1>(v));
    v = fmaxf(v, mt_dpp<0x4E>(v));
    return fmaxf(v, mt_dpp<0x141>(v));
}

// SPW super-blocks per wave (the wave's K slice), RT row tiles per workgroup.
// Per super-block the LDS region holds the A fragments [m = 2j + s][c][8
// halves] and, per group j, (sum of x, 2^(24 - s_j)) where 2^s_j is the
// group's power-of-two scale into f16 range.
template <int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_q4k(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                     int64_t tiles, const float *__restrict__ x,
                                                     float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    const int sb0 = w * SPW;
    int nsb = nb - sb0;
    nsb = nsb < 0 ? 0 : nsb > SPW ? SPW : nsb;
    uint8_t *wl = smem + w * SPW * MT_XBYTES;
    float *red = reinterpret_cast<float *>(smem + nw * SPW * MT_XBYTES);   // [nw][RT][64]
    const int64_t tile0 = (int64_t)blockIdx.x * RT;

    // ---- loads: x first (it is needed first), then every weight block ----
    float4 xv[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;
        const float4 v = *reinterpret_cast<const float4 *>(x + 256 * (int64_t)sb + 4 * lane);
        xv[k] = v;   // unconditional: fragments of k >= nsb are written but never read
    }
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

    // ---- x -> A fragments (hi/lo f16 of x * 2^s_j per group) + group data ----
    {
        const int j = lane >> 3, c = (lane & 7) >> 1;
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            const float4 v = xv[k];
            const float gs = mt_group8_sum((v.x + v.y) + (v.z + v.w));
            const float gmax = mt_group8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            int sh = 0;
            if (gmax > 0.0f && gmax <= 3.4e38f) {
                int e;
                frexpf(gmax, &e);
                sh = 15 - e;                  // group max * 2^sh in [2^14, 2^15)
                sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
            }
            const float up = ldexpf(1.0f, sh);
            uint8_t *frag = wl + k * MT_XBYTES;
            if ((lane & 7) == 7)
                reinterpret_cast<float2 *>(frag + 1024)[j] = make_float2(gs, ldexpf(1.0f, 24 - sh));
            const float a0 = v.x * up, a1 = v.y * up, a2 = v.z * up, a3 = v.w * up;
            const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1, h2 = (_Float16)a2, h3 = (_Float16)a3;
            const _Float16 l0 = (_Float16)(a0 - (float)h0), l1 = (_Float16)(a1 - (float)h1);
            const _Float16 l2 = (_Float16)(a2 - (float)h2), l3 = (_Float16)(a3 - (float)h3);
            *reinterpret_cast<h4 *>(frag + ((2 * j) * 4 + c) * 16 + (lane & 1) * 8) = h4{h0, h1, h2, h3};
            *reinterpret_cast<h4 *>(frag + ((2 * j + 1) * 4 + c) * 16 + (lane & 1) * 8) = h4{l0, l1, l2, l3};
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // ---- MFMA over (tile, super-block) ----
    mt_h8 a[8];
    const int m = lane & 15, q = lane >> 4, ga = m >> 1;
    uint32_t amask[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) amask[g] = ga == g ? ~0u : 0u;
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k >= nsb) break;
        const uint8_t *frag = wl + k * MT_XBYTES;
        const uint4 f = *reinterpret_cast<const uint4 *>(frag + (m * 4 + q) * 16);
        // lane's A fragment lives in a[m / 2] only; the other registers are zero
#pragma unroll
        for (int g = 0; g < 8; ++g) a[g] = mt_masked(f, amask[g]);
        // (sum, 2^(24 - s)) of groups 2q and 2q + 1
        const float4 gx = *reinterpret_cast<const float4 *>(frag + 1024 + 16 * q);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            mt_f4 dacc = mt_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < 8; ++g)
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[g], mt_b_q4k(q0[t][k], q1[t][k], g), dacc, 0, 0, 0);
            uint32_t sc0, sc1, mn0, mn1;
            kq_pair(hd[t][k], q, sc0, sc1, mn0, mn1);
            const float d = f16_to_f32(hd[t][k].x), dmin = f16_to_f32(hd[t][k].x >> 16);
            const float s = __builtin_fmaf((float)sc1 * 0.0625f * gx.w, dacc[2] + dacc[3],
                                           (float)sc0 * gx.y * (dacc[0] + dacc[1]));
            acc[t] = __builtin_fmaf(d, s, acc[t]);
            acc[t] = __builtin_fmaf(-dmin, __builtin_fmaf((float)mn0, gx.x, (float)mn1 * gx.z), acc[t]);
        }
    }
    // ---- reduce over the four lanes of a row and the waves, through LDS ----
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];
    __syncthreads();
    const int i = threadIdx.x;
    if (i < RT * 16) {
        const int t = i >> 4, n = i & 15;
        float s = 0.0f;
        for (int k = 0; k < nw; ++k) {
            const float *r = red + (k * RT + t) * 64 + n;
            s += (r[0] + r[16]) + (r[32] + r[48]);
        }
        const int64_t row = (tile0 + t) * MT_ROWS + n;
        if (tile0 + t < tiles && row < rows) y[row] = s;
    }
}

// ------------------------------------------------------------------- Q6_K
// MFMA t of a super-block covers natural values 32t .. 32t + 31 (half h =
// t / 4, quad c' = t % 4): q = ((ql >> 4 (c' / 2)) & 15) | ((qh >> 2c') & 3) << 4
// (engine/dequant.py:146-165), 0..63, as f16 subnormals. The block-diagonal A
// rows are (sub-block of the half jj = 0..7, split): value 32 (t % 4) + 8c + e
// of the half lies in sub-block 2 (t % 4) + c / 2, so lane (m, c) is nonzero
// in MFMA t only when m / 2 = 2 (t % 4) + c / 2, i.e. in A register a[m / 4].
// t6 is a compile-time constant after unrolling at every call site
__device__ __forceinline__ mt_h8 mt_b_q6k(int t6, uint4 ql_h, uint4 qh) {
    const int cq = t6 & 3, h = t6 >> 2;
    const uint32_t d0 = (cq & 1) ? ql_h.z : ql_h.x, d1 = (cq & 1) ? ql_h.w : ql_h.y;
    const uint32_t e0 = h ? qh.z : qh.x, e1 = h ? qh.w : qh.y;
    const uint32_t m0 = ((d0 >> (4 * (cq >> 1))) & 0x0F0F0F0Fu) | (((e0 >> (2 * cq)) & 0x03030303u) << 4);
    const uint32_t m1 = ((d1 >> (4 * (cq >> 1))) & 0x0F0F0F0Fu) | (((e1 >> (2 * cq)) & 0x03030303u) << 4);
    uint4 r;
    r.x = mt_lo_pair(m0);
    r.y = mt_hi_pair(m0);
    r.z = mt_lo_pair(m1);
    r.w = mt_hi_pair(m1);
    return __builtin_bit_cast(mt_h8, r);
}

__device__ __forceinline__ float mt_quad_sum(float v) {
    v += mt_dpp<0xB1>(v);
    return v + mt_dpp<0x4E>(v);
}
__device__ __forceinline__ float mt_quad_max(float v) {
    v = fmaxf(v, mt_dpp<0xB1>(v));
    return fmaxf(v, mt_dpp<0x4E>(v));
}

// Per super-block LDS: A fragments [half][jj][split][c & 1][8 halves] (1 KiB)
// and per sub-block (sum of x, 2^(24 - s)) (128 B).
template <int SPW, int RT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_mfma_q6k(const uint8_t *__restrict__ Wt, int64_t rows, int nb,
                                                      int64_t tiles, const float *__restrict__ x,
                                                      float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = lane_id(), w = wave_id(), nw = blockDim.x >> 6;
    const int sb0 = w * SPW;
    int nsb = nb - sb0;
    nsb = nsb < 0 ? 0 : nsb > SPW ? SPW : nsb;
    uint8_t *wl = smem + w * SPW * MT6_XBYTES;
    float *red = reinterpret_cast<float *>(smem + nw * SPW * MT6_XBYTES);   // [nw][RT][64]
    const int64_t tile0 = (int64_t)blockIdx.x * RT;

    float4 xv[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;
        const float4 v = *reinterpret_cast<const float4 *>(x + 256 * (int64_t)sb + 4 * lane);
        xv[k] = v;   // unconditional: fragments of k >= nsb are written but never read
    }
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

    // ---- x -> A fragments and sub-block data ----
    {
        const int h = lane >> 5, jj = (lane & 31) >> 2, cb = (lane & 3) >> 1;
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int k = 0; k < SPW; ++k) {
            const float4 v = xv[k];
            const float gs = mt_quad_sum((v.x + v.y) + (v.z + v.w));
            const float gmax = mt_quad_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            int sh = 0;
            if (gmax > 0.0f && gmax <= 3.4e38f) {
                int e;
                frexpf(gmax, &e);
                sh = 15 - e;
                sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
            }
            const float up = ldexpf(1.0f, sh);
            uint8_t *frag = wl + k * MT6_XBYTES;
            if ((lane & 3) == 0)
                reinterpret_cast<float2 *>(frag + 1024)[8 * h + jj] = make_float2(gs, ldexpf(1.0f, 24 - sh));
            const float a0 = v.x * up, a1 = v.y * up, a2 = v.z * up, a3 = v.w * up;
            const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1, h2 = (_Float16)a2, h3 = (_Float16)a3;
            const _Float16 l0 = (_Float16)(a0 - (float)h0), l1 = (_Float16)(a1 - (float)h1);
            const _Float16 l2 = (_Float16)(a2 - (float)h2), l3 = (_Float16)(a3 - (float)h3);
            const int base = ((h * 8 + jj) * 2) * 2 + cb;     // [h][jj][s][cb], s = 0
            *reinterpret_cast<h4 *>(frag + base * 16 + (lane & 1) * 8) = h4{h0, h1, h2, h3};
            *reinterpret_cast<h4 *>(frag + (base + 2) * 16 + (lane & 1) * 8) = h4{l0, l1, l2, l3};
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    mt_h8 a[4];
    const int m = lane & 15, q = lane >> 4, jj = m >> 1, sp = m & 1;
    const bool active = (q >> 1) == (jj & 1);
    uint32_t amask[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) amask[g] = (active && (jj >> 1) == g) ? ~0u : 0u;
    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        if (k >= nsb) break;
        const uint8_t *frag = wl + k * MT6_XBYTES;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 f = *reinterpret_cast<const uint4 *>(frag + ((((h * 8 + jj) * 2 + sp) * 2) + (q & 1)) * 16);
#pragma unroll
            for (int g = 0; g < 4; ++g) a[g] = mt_masked(f, amask[g]);
            // (sum, scale) of sub-blocks 8h + 2q and 8h + 2q + 1
            const float4 gx = *reinterpret_cast<const float4 *>(frag + 1024 + 8 * (8 * h + 2 * q));
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint4 qlh = h ? ql1[t][k] : ql0[t][k];
                mt_f4 dacc = mt_f4{0.0f, 0.0f, 0.0f, 0.0f};
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], mt_b_q6k(4 * h + 0, qlh, qh[t][k]), dacc, 0, 0, 0);
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], mt_b_q6k(4 * h + 1, qlh, qh[t][k]), dacc, 0, 0, 0);
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2], mt_b_q6k(4 * h + 2, qlh, qh[t][k]), dacc, 0, 0, 0);
                dacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[3], mt_b_q6k(4 * h + 3, qlh, qh[t][k]), dacc, 0, 0, 0);
                // int8 scales 8h + 2q, 8h + 2q + 1 of row n
                const uint32_t sw = (q >> 1) ? (h ? sc[t][k].w : sc[t][k].y) : (h ? sc[t][k].z : sc[t][k].x);
                const uint32_t s2 = sw >> (16 * (q & 1));
                const float sa = (float)(int8_t)(s2 & 0xFFu), sb = (float)(int8_t)((s2 >> 8) & 0xFFu);
                const float va = __builtin_fmaf(gx.y, dacc[0] + dacc[1], -32.0f * gx.x);
                const float vb = __builtin_fmaf(gx.w, dacc[2] + dacc[3], -32.0f * gx.z);
                acc[t] = __builtin_fmaf(f16_to_f32(dd[t][k]), __builtin_fmaf(sa, va, sb * vb), acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];
    __syncthreads();
    const int i = threadIdx.x;
    if (i < RT * 16) {
        const int t = i >> 4, n = i & 15;
        float s = 0.0f;
        for (int k = 0; k < nw; ++k) {
            const float *r = red + (k * RT + t) * 64 + n;
            s += (r[0] + r[16]) + (r[32] + r[48]);
        }
        const int64_t row = (tile0 + t) * MT_ROWS + n;
        if (tile0 + t < tiles && row < rows) y[row] = s;
    }
}

// Launch plan: the waves of a workgroup split the super-blocks. Rows of at
// most 32 super-blocks use up to 16 waves with SPW * RT <= 2 (short per-wave
// work keeps the latency chain of each wave short; 128 VGPRs suffice), longer
// rows up to 8 waves with SPW = ceil(nb / 8). Two row tiles per workgroup when
// that still gives about 4096 waves.
int launch_matvec_mfma(const lq_geom &g, const uint8_t *Wt, const float *x, float *y, hipStream_t s) {
    if (g.type != LQ_Q4_K && g.type != LQ_Q6_K) return fail(LOCALAI_ETYPE, "mfma matvec: Q4_K / Q6_K only");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(LOCALAI_EARG, "mfma matvec: x must be 16-byte aligned");
    const int nb = (int)g.nb;
    const bool q6 = g.type == LQ_Q6_K;
    const int64_t tiles = (g.rows + MT_ROWS - 1) / MT_ROWS;
    int spw = (nb + 15) / 16, waves, rt;
    bool big;
    if (spw <= 2) {
        waves = (nb + spw - 1) / spw;
        rt = (spw == 1 && tiles * waves >= 4096) ? 2 : 1;
        big = true;
    } else {
        spw = (nb + 7) / 8;
        waves = (nb + spw - 1) / spw;
        rt = 1;
        big = false;
    }
    if (spw > 8) return fail(LOCALAI_EARG, "mfma matvec: K too large (more than 16384 values)");
    dim3 grid((unsigned)((tiles + rt - 1) / rt)), block(64 * waves);
    const size_t lds = (size_t)waves * spw * (q6 ? MT6_XBYTES : MT_XBYTES) + (size_t)waves * rt * 64 * 4;
#define MT_L(S, R, M)                                                                                     \
    do {                                                                                                  \
        if (q6) hipLaunchKernelGGL((gemv_mfma_q6k<S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y); \
        else hipLaunchKernelGGL((gemv_mfma_q4k<S, R, M>), grid, block, lds, s, Wt, g.rows, nb, tiles, x, y);    \
    } while (0)
    if (big) {
        if (spw == 1 && rt == 2) MT_L(1, 2, 1024);
        else if (spw == 1) MT_L(1, 1, 1024);
        else MT_L(2, 1, 1024);
    } else {
        switch (spw) {
            case 3: MT_L(3, 1, 512); break;
            case 4: MT_L(4, 1, 512); break;
            case 5: MT_L(5, 1, 512); break;
            case 6: MT_L(6, 1, 512); break;
            case 7: MT_L(7, 1, 512); break;
            default: MT_L(8, 1, 512); break;
        }
    }
#undef MT_L
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
