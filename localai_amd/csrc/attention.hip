// The attention mixers of a decode step on the GPU: grouped-query attention
// of one token over the KV cache, and the gated delta-net recurrent step of
// Qwen3.5's linear-attention layers.
#include <hip/hip_runtime.h>

#include <cmath>

#include "dev_common.h"
#include "internal.h"

namespace lq {

// ---------------------------------------------------------------- GQA decode
//
// Counterpart of the decode step's attention, engine/model.py:222-227, and of
// Qwen3.5's full attention with its output gate, engine/qwen35.py:158-182.
// For query head h, with kv head h / G (G = n_heads / n_kv_heads; the
// np.repeat order of engine/model.py:225) and positions s in [start,
// position] (start = position + 1 - window under a sliding window, else 0):
//   score_s = (q_h . K[s]) / sqrt(head_dim),   p = softmax_s(score),
//   out_h   = sum_s p_s V[s]     (times sigmoid(gate_h) when a gate is given)
// after row `position` of K and V has been set to the token's k and v
// (engine/model.py:222). The caches are one layer of the reference's
// KVCache (engine/model.py:6-9): fp32 [max_seq, n_kv_heads, head_dim].
//
// Work layout: a workgroup of 4 waves owns one kv head and 16 RF positions,
// 4 RF per wave (head_dim = 64 NV). K is read 4 positions per load
// instruction, 16 lanes (one DPP row) per position, lane c holding 4
// consecutive floats of each 64-value piece; scores are summed across the row
// with DPP. V is read one position per instruction, lane l holding values
// NV l .. NV l + NV - 1, so p (broadcast from its position's row with
// readlane) weights a lane's own V values and o and l need no sums across
// lanes. Every K and V value of the chunk is requested up front and serves
// all G query heads of the kv head. Scores are kept in base-2 units
// (log2(e) / sqrt(head_dim) folded into the scale) so that p is one
// v_exp_f32; the chunk maximum crosses the wave's rows with gfx950's
// v_permlane16_swap / v_permlane32_swap, the waves meet in LDS. Each
// workgroup stores (o, max, l) per query head and
// attn_merge_kernel combines the chunks (split-sequence decode); with one
// chunk the workgroup writes the output itself. (A merge inside the same
// launch, by the last workgroup of each kv head, raised the chunk kernel's
// registers from about 110 to 255 per lane and was not faster.)

struct AttnArgs {
    const float *q, *k_new, *v_new, *gate;
    float *kc, *vc;
    int64_t position, start;
    int n_kv, hd, G;
    float scale;
    int nsplit;
    float *part;       // [n_kv, nsplit, G, hd + 2]: o[hd], max, l
    float *out;        // [n_heads, hd]
};

constexpr int ATTN_PIECE = 64;   // floats of a row piece (16 lanes x float4)
constexpr int ATTN_MC = 32;      // chunks a merge lane requests at once

// 1 / (1 + exp(-clip(x, -80, 80))), engine/qwen35.py:17-19
__device__ __forceinline__ float sigmoid_ref(float x) {
    return 1.0f / (1.0f + expf(-fminf(fmaxf(x, -80.0f), 80.0f)));
}

__device__ __forceinline__ float dot4(const float4 &a, const float4 &b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ uint32_t fbits(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float bitsf(uint32_t v) { return __builtin_bit_cast(float, v); }

// sum / max over each row of 16 lanes, the same value on every lane of the
// row: DPP quad xor 1, quad xor 2, half-row mirror, row mirror
__device__ __forceinline__ float row16_sum(float v) {
    v += bitsf(dpp_u32<0xB1>(fbits(v)));
    v += bitsf(dpp_u32<0x4E>(fbits(v)));
    v += bitsf(dpp_u32<0x141>(fbits(v)));
    v += bitsf(dpp_u32<0x140>(fbits(v)));
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, bitsf(dpp_u32<0xB1>(fbits(v))));
    v = fmaxf(v, bitsf(dpp_u32<0x4E>(fbits(v))));
    v = fmaxf(v, bitsf(dpp_u32<0x141>(fbits(v))));
    v = fmaxf(v, bitsf(dpp_u32<0x140>(fbits(v))));
    return v;
}

// v with lane l ^ 16 and l ^ 32 combined (the four rows of a wave), the same
// value on every lane: one swap of rows 0/1 and 2/3, then one of the halves
__device__ __forceinline__ float rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false);
    v = bitsf(a[0]) + bitsf(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
    return bitsf(b[0]) + bitsf(b[1]);
}
__device__ __forceinline__ float rows_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false);
    v = fmaxf(bitsf(a[0]), bitsf(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
    return fmaxf(bitsf(b[0]), bitsf(b[1]));
}

template <int N> struct AttnVec;
template <> struct AttnVec<1> { typedef float T; };
template <> struct AttnVec<2> { typedef float2 T; };
template <> struct AttnVec<4> { typedef float4 T; };

// N consecutive floats at p (16 N-byte aligned) into v[0..N)
template <int N>
__device__ __forceinline__ void ldv(const float *p, float (&v)[N]) {
    const typename AttnVec<N>::T t = *reinterpret_cast<const typename AttnVec<N>::T *>(p);
    __builtin_memcpy(&v[0], &t, sizeof(t));
}
// the same for cache rows, which a decode step reads once (nontemporal hint)
template <int N> struct AttnNt { typedef float T __attribute__((ext_vector_type(N))); };
template <> struct AttnNt<1> { typedef float T; };
template <int N>
__device__ __forceinline__ void ldv_nt(const float *p, float (&v)[N]) {
    const typename AttnNt<N>::T t = __builtin_nontemporal_load(reinterpret_cast<const typename AttnNt<N>::T *>(p));
    __builtin_memcpy(&v[0], &t, sizeof(t));
}
template <int N>
__device__ __forceinline__ void stv(float *p, const float (&v)[N]) {
    typename AttnVec<N>::T t;
    __builtin_memcpy(&t, &v[0], sizeof(t));
    *reinterpret_cast<typename AttnVec<N>::T *>(p) = t;
}

template <int NV, int GT, int RF>
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnArgs a) {
    constexpr int C = 16 * RF, P = 4 * RF;   // positions per workgroup / per wave
    __shared__ float red_m[4][GT], red_l[4][GT];
    __shared__ __attribute__((aligned(16))) float red_o[4][GT * NV * ATTN_PIECE];
    // kv head = workgroup index mod n_kv: workgroups go to the XCDs round
    // robin, so with 8 kv heads (or a multiple) each kv head's chunks, and the
    // merge workgroups of its query heads, share one XCD and its L2
    const int kh = (int)blockIdx.x % a.n_kv, split = (int)blockIdx.x / a.n_kv;
    const int wave = wave_id(), lane = lane_id(), pg = lane >> 4, c = lane & 15;
    const int hd = a.hd, G = a.G;
    const int64_t row = (int64_t)a.n_kv * hd;
    const int64_t s0 = a.start + (int64_t)split * C + P * wave;

    float4 qv[GT][NV];
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int j = 0; j < NV; ++j)
            // heads past G (kernel sized for more) repeat head G - 1; their
            // results are never stored
            qv[g][j] = ld4(a.q + (int64_t)(kh * G + (g < G ? g : G - 1)) * hd + ATTN_PIECE * j + 4 * c);

    // every K and V value of the wave's P positions requested before any is
    // used (the token's own row from k_new / v_new); rows past `position` are
    // not read. K: row r of 4 positions, 16 lanes per position, lane c holds
    // values 64 j + 4 c ..; V: position i, lane l holds values NV l .. NV l + NV - 1.
    float4 kv[RF][NV];
    bool valid[RF];
#pragma unroll
    for (int r = 0; r < RF; ++r) {
        const int64_t s = s0 + 4 * r + pg;
        valid[r] = s <= a.position;
        const bool own = s == a.position && a.k_new;
        const float *kp = own ? a.k_new + (int64_t)kh * hd : a.kc + (valid[r] ? s : a.start) * row + (int64_t)kh * hd;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float t[4];
            ldv_nt<4>(kp + ATTN_PIECE * j + 4 * c, t);
            kv[r][j] = make_float4(t[0], t[1], t[2], t[3]);
        }
    }
    float vv[P][NV];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int64_t s = s0 + i;
        const bool own = s == a.position && a.k_new;
        const float *vp = own ? a.v_new + (int64_t)kh * hd
                              : a.vc + (s <= a.position ? s : a.start) * row + (int64_t)kh * hd;
        ldv_nt<NV>(vp + NV * lane, vv[i]);
    }
    // scores in base-2 units (scale = log2(e) / sqrt(head_dim)): the 16
    // lanes of a position each hold 4 NV products
    float sc[RF][GT];
#pragma unroll
    for (int r = 0; r < RF; ++r)
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < NV; ++j) d += dot4(qv[g][j], kv[r][j]);
            d = row16_sum(d);
            sc[r][g] = valid[r] ? d * a.scale : -INFINITY;
        }

    // chunk maximum per head: the wave's rounds, its four rows, the four waves
    float mx[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        float m = sc[0][g];
#pragma unroll
        for (int r = 1; r < RF; ++r) m = fmaxf(m, sc[r][g]);
        m = rows_max(m);
        if (lane == 0) red_m[wave][g] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GT; ++g)
        mx[g] = fmaxf(fmaxf(red_m[0][g], red_m[1][g]), fmaxf(red_m[2][g], red_m[3][g]));

    // p = 2^(score - max) (masked rows 0), broadcast per position from its
    // row; l and the p-weighted V rows in each lane's own values
    float acc[GT][NV], ls[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        ls[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < NV; ++e) acc[g][e] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < RF; ++r)
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const float p = valid[r] ? __builtin_amdgcn_exp2f(sc[r][g] - mx[g]) : 0.0f;
            ls[g] += p;     // the lane's own row; the rows are summed below
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float pb = uniform_f(p, 16 * q4);
#pragma unroll
                for (int e = 0; e < NV; ++e) acc[g][e] += pb * vv[4 * r + q4][e];
            }
        }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        const float l = rows_sum(ls[g]);
        if (lane == 0) red_l[wave][g] = l;
        stv<NV>(&red_o[wave][g * NV * ATTN_PIECE + NV * lane], acc[g]);
    }
    __syncthreads();

    // the token's row goes into the cache (no other workgroup reads it);
    // last, so that no wait for its values comes before the arithmetic
    if (a.k_new && a.position >= s0 && a.position < s0 + P) {
        const int64_t off = a.position * row + (int64_t)kh * hd;
#pragma unroll
        for (int r = 0; r < RF; ++r)
            if (s0 + 4 * r + pg == a.position)
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    *reinterpret_cast<float4 *>(a.kc + off + ATTN_PIECE * j + 4 * c) = kv[r][j];
#pragma unroll
        for (int i = 0; i < P; ++i)
            if (s0 + i == a.position) stv<NV>(a.vc + off + NV * lane, vv[i]);
    }

    // the workgroup's sums over its 4 waves; thread i handles values i, i + 256, ...
    const int nval = G * hd;
    const int64_t rec = hd + 2;
    float *pw = a.part + ((int64_t)kh * a.nsplit + split) * G * rec;
    for (int i = threadIdx.x; i < nval; i += 256) {
        const int g = i / hd, d = i % hd;
        const int o = g * NV * ATTN_PIECE + d;
        const float ov = (red_o[0][o] + red_o[1][o]) + (red_o[2][o] + red_o[3][o]);
        const float lv = (red_l[0][g] + red_l[1][g]) + (red_l[2][g] + red_l[3][g]);
        if (a.nsplit == 1) {
            const int64_t h = (int64_t)kh * G + g;
            float y = ov / lv;
            if (a.gate) y *= sigmoid_ref(a.gate[h * hd + d]);
            a.out[h * hd + d] = y;
        } else {
            pw[g * rec + d] = ov;
            if (d == 0) {
                pw[g * rec + hd] = fmaxf(fmaxf(red_m[0][g], red_m[1][g]), fmaxf(red_m[2][g], red_m[3][g]));
                pw[g * rec + hd + 1] = lv;
            }
        }
    }
}

// Merge of the chunks: workgroup (x, b) writes values 64 b .. 64 b + 63 of
// query head h = (x mod n_kv) G + x / n_kv. With M the largest chunk maximum (base-2 units), out =
// sum_i 2^(m_i - M) o_i / sum_i 2^(m_i - M) l_i. The workgroup's waves split
// the chunks ATTN_MC at a time (wave w: chunks 32 w, 32 (w + nw), ...), so a
// lane requests its ATTN_MC chunk values and the chunks' (max, l) in one round;
// each wave keeps a running maximum, its weights reach the lanes by readlane,
// and the waves meet in LDS.
__global__ __launch_bounds__(512) void attn_merge_kernel(AttnArgs a) {
    __shared__ float red_m[8], red_l[8], red_o[8][64];
    // the kv head is the workgroup index mod n_kv, as in the chunk kernel
    const int kh = (int)blockIdx.x % a.n_kv, g = (int)blockIdx.x / a.n_kv, h = kh * a.G + g, hd = a.hd, ns = a.nsplit;
    const int lane = lane_id(), wave = wave_id(), nw = (int)(blockDim.x >> 6);
    const int d = 64 * blockIdx.y + lane;
    const int64_t rec = hd + 2, stride = (int64_t)a.G * rec;
    const float *base = a.part + (int64_t)kh * ns * stride + g * rec;
    float M = -INFINITY, o = 0.0f, l = 0.0f;
    for (int c0 = ATTN_MC * wave; c0 < ns; c0 += ATTN_MC * nw) {
        const int cn = ns - c0 < ATTN_MC ? ns - c0 : ATTN_MC;
        const float *pc = base + (int64_t)c0 * stride;
        const int li = lane < cn ? lane : 0;
        const float mi = lane < cn ? pc[li * stride + hd] : -INFINITY;
        const float lv = lane < cn ? pc[li * stride + hd + 1] : 0.0f;
        float v[ATTN_MC];
#pragma unroll
        for (int i = 0; i < ATTN_MC; ++i) v[i] = pc[(i < cn ? i : 0) * stride + d];
        const float Mn = fmaxf(M, rows_max(row16_max(mi)));
        const float f = __builtin_amdgcn_exp2f(M - Mn);   // 0 on the first pass (M = -inf)
        const float w = lane < cn ? __builtin_amdgcn_exp2f(mi - Mn) : 0.0f;
        float oc = 0.0f;
#pragma unroll
        for (int i = 0; i < ATTN_MC; ++i) oc += uniform_f(w, i) * v[i];
        o = o * f + oc;
        l = l * f + rows_sum(row16_sum(w * lv));
        M = Mn;
    }
    red_o[wave][lane] = o;
    if (lane == 0) {
        red_m[wave] = M;
        red_l[wave] = l;
    }
    __syncthreads();
    if (wave == 0) {
        float Mw = -INFINITY;
        for (int w = 0; w < nw; ++w) Mw = fmaxf(Mw, red_m[w]);
        float ov = 0.0f, lt = 0.0f;
        for (int w = 0; w < nw; ++w) {
            // a wave without chunks holds m = -inf and zero sums
            const float f = red_m[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w] - Mw);
            ov += f * red_o[w][lane];
            lt += f * red_l[w];
        }
        float y = ov / lt;
        if (a.gate) y *= sigmoid_ref(a.gate[(int64_t)h * hd + d]);
        a.out[(int64_t)h * hd + d] = y;
    }
}

// rounds of 4 positions per wave: all of a chunk's K / V stays in registers
// next to the query and accumulator values (GT NV <= 16)
constexpr int attn_rounds(int nv, int gt) { return gt * nv <= 8 ? 4 : 2; }

static int attn_shape(int hd, int G, int *nv, int *gt) {
    if (hd % ATTN_PIECE || hd / ATTN_PIECE < 1 || hd / ATTN_PIECE > 4 || hd / ATTN_PIECE == 3) return 1;
    *nv = hd / ATTN_PIECE;
    *gt = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 0;
    if (!*gt || *gt * *nv > 16) return 1;
    return 0;
}

size_t attention_workspace_bytes(int64_t max_seq, int n_heads, int n_kv, int hd) {
    const int G = n_heads / n_kv;
    int nv, gt;
    if (attn_shape(hd, G, &nv, &gt)) return 0;
    const int C = 16 * attn_rounds(nv, gt);
    const int64_t nsplit = (max_seq + C - 1) / C;
    return (size_t)((int64_t)n_kv * nsplit * G * (hd + 2) * 4);
}

int launch_attention_decode(const float *q, const float *k_new, const float *v_new, float *kc, float *vc,
                            int64_t position, int64_t window, int n_heads, int n_kv, int hd, const float *gate,
                            float *out, void *ws, int64_t ws_bytes, hipStream_t s) {
    AttnArgs a{};
    a.G = n_heads / n_kv;
    int nv, gt;
    if (attn_shape(hd, a.G, &nv, &gt))
        return fail(LOCALAI_ETYPE, "attention: head_dim 64, 128 or 256 and at most 16 / (head_dim / 64) query "
                                   "heads per kv head");
    const int C = 16 * attn_rounds(nv, gt);
    a.q = q; a.k_new = k_new; a.v_new = v_new; a.gate = gate; a.kc = kc; a.vc = vc;
    a.position = position;
    a.start = window > 0 && position + 1 - window > 0 ? position + 1 - window : 0;
    a.n_kv = n_kv; a.hd = hd;
    a.scale = (float)(1.4426950408889634 / std::sqrt((double)hd));   // log2(e) / sqrt(head_dim)
    const int64_t len = position - a.start + 1, nsplit = (len + C - 1) / C;
    if (nsplit > 65535) return fail(LOCALAI_EARG, "attention: too many positions");
    a.nsplit = (int)nsplit;
    a.part = (float *)ws;
    a.out = out;
    if (nsplit > 1 && (!ws || ws_bytes < (int64_t)n_kv * nsplit * a.G * (hd + 2) * 4))
        return fail(LOCALAI_EARG, "attention: workspace too small");
    const dim3 grid((unsigned)(nsplit * n_kv));
#define LQ_ATT(NV, GT)                                                                                        \
    if (nv == NV && gt == GT) {                                                                               \
        hipLaunchKernelGGL((attn_chunk_kernel<NV, GT, attn_rounds(NV, GT)>), grid, dim3(256), 0, s, a);       \
    }
    LQ_ATT(1, 1) else LQ_ATT(1, 2) else LQ_ATT(1, 4) else LQ_ATT(1, 8)
    else LQ_ATT(2, 1) else LQ_ATT(2, 2) else LQ_ATT(2, 4) else LQ_ATT(2, 8)
    else LQ_ATT(4, 1) else LQ_ATT(4, 2) else LQ_ATT(4, 4)
#undef LQ_ATT
    LQ_HIP(hipGetLastError());
    if (nsplit > 1) {
        const int nw = (int)((nsplit + ATTN_MC - 1) / ATTN_MC < 8 ? (nsplit + ATTN_MC - 1) / ATTN_MC : 8);
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)n_heads, (unsigned)((hd + 63) / 64)), dim3(64 * nw), 0,
                           s, a);
        LQ_HIP(hipGetLastError());
    }
    return LOCALAI_OK;
}

// ---------------------------------------------------------------- delta net
//
// Counterpart of delta_net_step (engine/numba_kernels.py:11-45), the gated
// delta-rule recurrent step of Qwen3.5's linear attention
// (engine/qwen35.py:224-252). Per head h, with state S [key_dim, value_dim]:
//   S *= exp(decay[h]);  pred = S^T k;  delta = (v - pred) * beta[h]
//   S += k delta^T;      core = S^T q
// Column vi of S goes through the reference loop's exact float32
// operations: each product and each sum rounded on its own (no fused
// multiply-add), the sums in ki ascending order, so state and core equal the
// reference loop's bit for bit given the same factor exp(decay). The factor
// here is the fp64 exponential rounded once to fp32 (correctly rounded); the
// reference's np.exp on float32 can differ from it in the last bit or two.
//
// delta_net_kernel (key_dim KF, 64 or 128): a workgroup of 4 waves owns 64
// value columns of one head; lane = column. Only the two sums are serial, so
// only they stay on one wave: each wave scales its own rows of the slab (rows
// 4 at a time, interleaved over the waves), keeps them in registers, and
// writes the products keep * k to LDS; wave 0 adds them in ki order (128
// dependent adds, the products read 4 at a time); then each wave forms its
// rows' updated values, stores them and writes val * q; wave 0 adds those.
// Every product and sum is the reference loop's own fp32 operation.
// delta_net_any_kernel: any key_dim, one wave per 64 columns straight from
// global memory.
template <int KF>
__global__ __launch_bounds__(256) void delta_net_kernel(float *__restrict__ state, const float *__restrict__ q,
                                                        const float *__restrict__ k, const float *__restrict__ v,
                                                        const float *__restrict__ decay,
                                                        const float *__restrict__ beta, float *__restrict__ core,
                                                        int VD) {
#pragma clang fp contract(off)
    constexpr int RW = KF / 4, LD = KF + 4;  // rows per wave; padded column stride of the product table
    __shared__ __align__(16) float prod[64 * LD];
    __shared__ float delta_s[64];
    const int h = blockIdx.y, c0 = blockIdx.x * 64, tid = (int)threadIdx.x, col = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: k and q by scalar loads
    const bool in = c0 + col < VD;
    // columns past VD read column c0 and store nothing
    float *hs = state + (int64_t)h * KF * VD + c0 + (in ? col : 0);
    const float *kh = k + (int64_t)h * KF, *qh = q + (int64_t)h * KF;
    float keep[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) keep[i] = hs[(int64_t)(16 * (i >> 2) + 4 * w + (i & 3)) * VD];
    const float factor = (float)exp((double)decay[h]);
    float *mine = prod + col * LD + 4 * w;
#pragma unroll
    for (int i = 0; i < RW; i += 4) {
        float4 pr;
        float *pp = &pr.x;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            keep[i + j] = keep[i + j] * factor;
            pp[j] = keep[i + j] * kh[16 * (i >> 2) + 4 * w + j];
        }
        *reinterpret_cast<float4 *>(mine + 16 * (i >> 2)) = pr;
    }
    __syncthreads();
    if (w == 0) {
        float pred = 0.0f;
#pragma unroll
        for (int ki = 0; ki < KF; ki += 4) {
            const float4 pr = *reinterpret_cast<const float4 *>(prod + col * LD + ki);
            pred = pred + pr.x;
            pred = pred + pr.y;
            pred = pred + pr.z;
            pred = pred + pr.w;
        }
        delta_s[col] = in ? (v[(int64_t)h * VD + c0 + col] - pred) * beta[h] : 0.0f;
    }
    __syncthreads();
    const float delta = delta_s[col];
#pragma unroll
    for (int i = 0; i < RW; i += 4) {
        float4 pr;
        float *pp = &pr.x;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ki = 16 * (i >> 2) + 4 * w + j;
            keep[i + j] = keep[i + j] + kh[ki] * delta;
            pp[j] = keep[i + j] * qh[ki];
        }
        *reinterpret_cast<float4 *>(mine + 16 * (i >> 2)) = pr;
    }
    if (in)
#pragma unroll
        for (int i = 0; i < RW; ++i) hs[(int64_t)(16 * (i >> 2) + 4 * w + (i & 3)) * VD] = keep[i];
    __syncthreads();
    if (w == 0 && in) {
        float acc = 0.0f;
#pragma unroll
        for (int ki = 0; ki < KF; ki += 4) {
            const float4 pr = *reinterpret_cast<const float4 *>(prod + col * LD + ki);
            acc = acc + pr.x;
            acc = acc + pr.y;
            acc = acc + pr.z;
            acc = acc + pr.w;
        }
        core[(int64_t)h * VD + c0 + col] = acc;
    }
}

__global__ __launch_bounds__(64) void delta_net_any_kernel(float *__restrict__ state, const float *__restrict__ q,
                                                           const float *__restrict__ k, const float *__restrict__ v,
                                                           const float *__restrict__ decay,
                                                           const float *__restrict__ beta, float *__restrict__ core,
                                                           int KD, int VD) {
#pragma clang fp contract(off)
    const int h = blockIdx.y, vi = blockIdx.x * 64 + (int)threadIdx.x;
    if (vi >= VD) return;
    const float factor = (float)exp((double)decay[h]);
    float *col = state + (int64_t)h * KD * VD + vi;
    const float *kh = k + (int64_t)h * KD, *qh = q + (int64_t)h * KD;
    float pred = 0.0f, acc = 0.0f;
    for (int ki = 0; ki < KD; ++ki) {
        const float val = col[(int64_t)ki * VD] * factor;
        col[(int64_t)ki * VD] = val;
        pred = pred + val * kh[ki];
    }
    const float delta = (v[(int64_t)h * VD + vi] - pred) * beta[h];
    for (int ki = 0; ki < KD; ++ki) {
        const float val = col[(int64_t)ki * VD] + kh[ki] * delta;
        col[(int64_t)ki * VD] = val;
        acc = acc + val * qh[ki];
    }
    core[(int64_t)h * VD + vi] = acc;
}

int launch_delta_net(float *state, const float *q, const float *k, const float *v, const float *decay,
                     const float *beta, float *core, int heads, int KD, int VD, hipStream_t s) {
    const dim3 grid((unsigned)((VD + 63) / 64), (unsigned)heads);
    if (KD == 128)
        hipLaunchKernelGGL(delta_net_kernel<128>, grid, dim3(256), 0, s, state, q, k, v, decay, beta, core, VD);
    else if (KD == 64)
        hipLaunchKernelGGL(delta_net_kernel<64>, grid, dim3(256), 0, s, state, q, k, v, decay, beta, core, VD);
    else
        hipLaunchKernelGGL(delta_net_any_kernel, grid, dim3(64), 0, s, state, q, k, v, decay, beta, core, KD, VD);
    LQ_HIP(hipGetLastError());
    return LOCALAI_OK;
}

}  // namespace lq
