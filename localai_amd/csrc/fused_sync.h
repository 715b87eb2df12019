// fused_sync.h -- hand-offs between the workgroups of one launch (the fused
// one-token MoE layer): a counter block in device memory, device-coherent
// loads and stores, bounded waits.
#pragma once
#include "dev_common.h"

namespace lq {

// Counter block of the fused one-token expert kernel (moe_decode1_kernel),
// in the workspace, zero when the launch starts:
// D1_NCNT gate_up completion counters (gate_up tile r counts on r % D1_NCNT,
// so no counter takes more than a few dozen atomics), a counter of full
// counters, the all-done flag the down tiles poll, and an error word, each
// on a 128-byte line of its own.
constexpr int D1_NCNT = 16, D1_LINE = 32;
enum {
    D1_FULL = D1_NCNT * D1_LINE,
    D1_DONE = D1_FULL + D1_LINE,
    D1_ERROR = D1_DONE + D1_LINE,
    D1_WORDS = D1_ERROR + D1_LINE
};

// Default bound on every wait of the fused layer (polls, seconds in all): a
// wait that runs out sets D1_ERR_WAIT in the error word and its workgroup
// adds NaN to its rows of the output, so the failure shows in the result and
// the host can read the word afterwards (localai_hip_moe_error).
constexpr int D1_SPIN_LIMIT = 1 << 22;
// Bits of the error word
constexpr uint32_t D1_ERR_WAIT = 1u;    // a wait for the gate_up tiles ran out
constexpr uint32_t D1_ERR_INDEX = 2u;   // an expert index outside [0, E) that is not the skip route

__device__ __forceinline__ void d1_error(uint32_t *sync, uint32_t bit) {
    __hip_atomic_fetch_or(sync + D1_ERROR, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Data handed between workgroups of the fused layer moves with device-
// coherent (relaxed, device-scope atomic) loads and stores, which bypass the
// per-XCD caches; a store of a flag follows the data stores' completion
// (vmcnt(0)). No acquire or release fences: on this GPU each would
// invalidate or write back a whole XCD's L2.
template <typename V>
__device__ __forceinline__ V d1_get(const V *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ void d1_put(V *p, V v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void d1_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Whole workgroup: wait until the all-done flag is set. One thread polls: a
// first sleep of about 8000 cycles (the gate_up tiles take several times
// that), then about 1000 cycles between polls, at most `spin` polls; the
// others wait at the barrier. false: the wait ran out (D1_ERR_WAIT is set).
// flag: one int of LDS.
__device__ __forceinline__ bool d1_wait_done(uint32_t *sync, int *flag, int spin) {
    if (threadIdx.x == 0) {
        int ok = 0;
        __builtin_amdgcn_s_sleep(127);
        for (int n = 0; n < spin; ++n) {
            if (d1_get(sync + D1_DONE) != 0u) {
                ok = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(15);
        }
        if (!ok) d1_error(sync, D1_ERR_WAIT);
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

// Workgroup r of n (one thread): count it done. The one that fills its
// counter (its share: the r' < n with r' % D1_NCNT == r % D1_NCNT) counts a
// full counter; the one that fills the last counter sets the flag and
// returns true.
__device__ __forceinline__ bool d1_count(uint32_t *sync, int r, int n) {
    const int c = r % D1_NCNT;
    const uint32_t share = (uint32_t)((n - c + D1_NCNT - 1) / D1_NCNT);
    const int ncnt = n < D1_NCNT ? n : D1_NCNT;
    const uint32_t before =
        __hip_atomic_fetch_add(sync + c * D1_LINE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before + 1 == share) {
        const uint32_t full =
            __hip_atomic_fetch_add(sync + D1_FULL, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (full + 1 == (uint32_t)ncnt) {
            d1_put(sync + D1_DONE, 1u);
            return true;
        }
    }
    return false;
}

// x of the wave's super-blocks (as mt_load_x) with device-coherent loads
template <int SPW>
__device__ __forceinline__ void d1_load_x(float4 (&xv)[SPW], const float *x, int nb, int sb0, int lane) {
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        const int sb = sb0 + k < nb ? sb0 + k : nb - 1;
        const uint64_t *p = reinterpret_cast<const uint64_t *>(x + 256 * (int64_t)sb + 4 * lane);
        const uint64_t lo = d1_get(p), hi = d1_get(p + 1);
        xv[k] = make_float4(__builtin_bit_cast(float, (uint32_t)lo), __builtin_bit_cast(float, (uint32_t)(lo >> 32)),
                            __builtin_bit_cast(float, (uint32_t)hi), __builtin_bit_cast(float, (uint32_t)(hi >> 32)));
    }
}

}  // namespace lq
