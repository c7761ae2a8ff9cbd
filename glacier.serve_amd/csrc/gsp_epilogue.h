// Epilogue shared by the decode kernels: merge the four waves of a workgroup
// through LDS, then either write the normalised output (unsplit unit) or
// publish a (max, sum, unnormalised out) partial and, in the last split of a
// (query token, KV head) pair to finish, merge all partials with the
// log-sum-exp rescale (FlashDecoding-style split-KV).
//
// Cross-workgroup visibility uses agent-scope relaxed atomic accesses, which
// gfx950 issues as `global_store/global_load ... sc1` (coherent across the
// XCDs' L2s), plus an explicit wait for the stores to complete before the
// pair's counter is bumped.  No device-scope fence is used: on this part a
// release fence writes back the whole L2 of the XCD.  The last split resets
// the counter, so counters are zero between launches.  Nothing spins.
#pragma once

#include "gsp_internal.h"

namespace gsp {

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): every vector memory access of
// this wave, stores included, has completed.
__device__ __forceinline__ void wait_vm_complete() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// LDS of the epilogue.  `o`, `m`, `l` hold the four waves' states; `w` holds
// the per-split merge weights of the last split.
template <int D, int GMAX>
struct EpilogueLds {
    float o[kDecodeWaves][GMAX][D];
    float m[kDecodeWaves][GMAX];
    float l[kDecodeWaves][GMAX];
    float w[kMaxSplits][GMAX];
    float lsum[kMaxSplits][GMAX];
    int last;
};

template <int D, int GMAX>
__device__ __forceinline__ void finish_unit(const DecodeArgs& a, const DecodeUnit& u, int G,
                                            EpilogueLds<D, GMAX>& sh) {
    const int tid = threadIdx.x;
    const int h0 = u.kvh * G;
    const int split = u.split_info & 0xFFFF;
    const int nsplit = u.split_info >> 16;
    const int64_t pair = (int64_t)u.slot;  // first partial slot of the pair (-1: unsplit)

    // Merge the four waves; a wave without pages has m = -inf and weighs 0.
    for (int idx = tid; idx < G * D; idx += kDecodeThreads) {
        const int g = idx / D;
        const int e = idx - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, sh.m[w][g]);
        float L = 0.f;
        float O = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            const float f = fast_exp2(sh.m[w][g] - M);
            L = fmaf(sh.l[w][g], f, L);
            O = fmaf(sh.o[w][g][e], f, O);
        }
        if (nsplit == 1) {
            a.out[((int64_t)u.qi * a.n_heads + h0 + g) * D + e] = O / L;
        } else {
            const int64_t ps = (pair + split) * G + g;
            coherent_store(a.part_o + ps * D + e, O);
            if (e == 0) {
                coherent_store(a.part_ml + ps * 2 + 0, M);
                coherent_store(a.part_ml + ps * 2 + 1, L);
            }
        }
    }
    if (nsplit == 1) return;

    wait_vm_complete();
    __syncthreads();
    if (tid == 0) {
        int* ctr = a.counters + (int64_t)u.qi * a.n_kv + u.kvh;
        const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = (prev == nsplit - 1);
    }
    __syncthreads();
    if (!sh.last) return;

    // Last split of the pair: weights w_s = 2^(m_s - M) / sum_s' 2^(m_s' - M) l_s'.
    for (int idx = tid; idx < nsplit * G; idx += kDecodeThreads) {
        const int s = idx / G;
        const int g = idx - s * G;
        const int64_t ps = (pair + s) * G + g;
        sh.w[s][g] = coherent_load(a.part_ml + ps * 2 + 0);
        sh.lsum[s][g] = coherent_load(a.part_ml + ps * 2 + 1);
    }
    __syncthreads();
    if (tid < G) {
        const int g = tid;
        float M = -INFINITY;
        for (int s = 0; s < nsplit; ++s) M = fmaxf(M, sh.w[s][g]);
        float L = 0.f;
        for (int s = 0; s < nsplit; ++s) {
            const float f = fast_exp2(sh.w[s][g] - M);
            sh.w[s][g] = f;
            L = fmaf(sh.lsum[s][g], f, L);
        }
        const float inv = 1.0f / L;
        for (int s = 0; s < nsplit; ++s) sh.w[s][g] *= inv;
    }
    __syncthreads();
    for (int idx = tid; idx < G * D; idx += kDecodeThreads) {
        const int g = idx / D;
        const int e = idx - g * D;
        const float* po = a.part_o + (pair * G + g) * D + e;
        const int64_t stride = (int64_t)G * D;
        float O0 = 0.f, O1 = 0.f, O2 = 0.f, O3 = 0.f;
        int s = 0;
        for (; s + 4 <= nsplit; s += 4) {
            O0 = fmaf(coherent_load(po + (s + 0) * stride), sh.w[s + 0][g], O0);
            O1 = fmaf(coherent_load(po + (s + 1) * stride), sh.w[s + 1][g], O1);
            O2 = fmaf(coherent_load(po + (s + 2) * stride), sh.w[s + 2][g], O2);
            O3 = fmaf(coherent_load(po + (s + 3) * stride), sh.w[s + 3][g], O3);
        }
        for (; s < nsplit; ++s) O0 = fmaf(coherent_load(po + s * stride), sh.w[s][g], O0);
        a.out[((int64_t)u.qi * a.n_heads + h0 + g) * D + e] = (O0 + O1) + (O2 + O3);
    }
    if (tid == 0) {
        __hip_atomic_store(a.counters + (int64_t)u.qi * a.n_kv + u.kvh, 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace gsp
