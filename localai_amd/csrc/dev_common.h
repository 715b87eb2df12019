// Device-side helpers shared by the kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qformat.h"

namespace lq {

typedef float lq_f4 __attribute__((ext_vector_type(4)));   // one 16-byte register tuple

// IEEE binary16 -> binary32 by the hardware conversion (one instruction):
// exact for every finite value and both infinities; a signalling NaN comes
// out quiet. Used where the value only feeds arithmetic (matvec / GEMM scales).
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
    return (float)h;
}

// IEEE binary16 -> binary32 keeping NaN payloads bit for bit (a signalling
// NaN stays signalling): sign | 0x7f800000 | mantissa << 13, as half_to_float
// does (engine/native_quant.cpp:12-33) and as NumPy's '<f2' widening does
// (engine/dequant.py:20-24). Every other input takes the hardware conversion,
// which is exact for them. Used by the dequant kernels, whose outputs are
// compared bit for bit.
__device__ __forceinline__ float f16_to_f32_bits(uint32_t bits16) {
    const uint32_t h = bits16 & 0xffffu;
    const float f = f16_to_f32(h);
    const uint32_t nan = ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13);
    return (h & 0x7c00u) == 0x7c00u && (h & 0x3ffu) ? __builtin_bit_cast(float, nan) : f;
}

// Byte i of a dword as float: each maps to one v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float ubyte0(uint32_t v) { return (float)(v & 0xffu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return (float)((v >> 8) & 0xffu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return (float)((v >> 16) & 0xffu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return (float)(v >> 24); }

// A constant the compiler cannot see through (materialised in an SGPR). Used
// for nibble masks: with a visible constant mask the compiler narrows each
// byte conversion into a bitfield extract plus ubyte0 conversion (two
// instructions per value instead of one).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    uint32_t r;
    asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}

__device__ __forceinline__ uint32_t u4_get(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Sum over aligned groups of G consecutive lanes (G = 2..64); every lane of a
// group receives the group sum. Butterfly over lane xor masks 1, 2, ..., G/2.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

template <int G>
__device__ __forceinline__ double group_sum_f64(double v) {
#pragma unroll
    for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float uniform_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Wave-wide max / min, on every lane: DPP inside each row of 16 lanes (quad
// xor 1, quad xor 2, half-row mirror, row mirror), then the four rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return max(max(a, b), max(c, d));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(v));
    v = min(v, dpp_u32<0x4E>(v));
    v = min(v, dpp_u32<0x141>(v));
    v = min(v, dpp_u32<0x140>(v));
    const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return min(min(a, b), min(c, d));
}

__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// g / (1 + exp(-clip(g, -80, 80))), engine/zaya.py:305
__device__ __forceinline__ float silu(float g) {
    const float c = fminf(fmaxf(g, -80.0f), 80.0f);
    return g / (1.0f + expf(-c));
}

// silu with the hardware exponential and reciprocal (a few ulp), for
// epilogues of the f16-operand GEMMs, whose own error is ~2^-12
__device__ __forceinline__ float silu_fast(float g) {
    const float c = fminf(fmaxf(g, -80.0f), 80.0f);
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-c));
}

}  // namespace lq
