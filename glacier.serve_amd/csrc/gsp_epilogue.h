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

// The query heads one decode workgroup serves for a unit's KV head.  A GQA
// group of up to 16 heads is one tile; a larger group is cut into tiles of 16
// (the last one smaller), one per grid.y, each with its own partials and
// counters.  dv is the output width (v_head_dim); the partials of a tile are
// [slot][gs][dv] and [slot][gs][2], its counters [total_q][n_kv].
struct Tile {
    int G;              // heads in this tile
    int hoff;           // first head of the tile within its KV head's group
    int gs;             // heads per partial slot
    int dv;             // output width
    float* part_o;
    float* part_ml;
    int32_t* counters;
};

// LDS of the epilogue: the four waves' states (rows of D >= dv floats).
template <int D, int GMAX>
struct EpilogueLds {
    float o[kDecodeWaves][GMAX][D];
    float m[kDecodeWaves][GMAX];
    float l[kDecodeWaves][GMAX];
    int last;      // the pair counted last is complete: merge it
    int last_pub;  // the same, for a second pair settled after a workgroup's final unit
};

// Splits merged per round trip by the last split of a pair.
constexpr int kMergeChunk = 8;

__device__ __forceinline__ float* out_row(const DecodeArgs& a, const DecodeUnit& u, const Tile& t, int g) {
    return a.out + ((int64_t)u.qi * a.n_heads + (int64_t)u.kvh * a.group + t.hoff + g) * t.dv;
}

// Merges the four waves' states (LDS) of unit u and writes the result: the
// normalised output of an unsplit unit, or the (max, sum, unnormalised out)
// partial of a split piece, stored coherently.  Nothing here waits for the
// stores; the caller orders them before the pair's counter is bumped.
template <int D, int GMAX>
__device__ __forceinline__ void publish_unit(const DecodeArgs& a, const DecodeUnit& u, const Tile& t,
                                             EpilogueLds<D, GMAX>& sh) {
    const int tid = threadIdx.x;
    const int G = t.G;
    const int dv = t.dv;
    const int split = u.split_info & 0xFFFF;
    const int nsplit = u.split_info >> 16;
    const int64_t pair = (int64_t)u.slot;  // first partial slot of the pair (-1: unsplit)

    // A wave without pages has m = -inf and weighs 0.
    for (int idx = tid; idx < G * dv; idx += kDecodeThreads) {
        const int g = idx / dv;
        const int e = idx - g * dv;
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
            out_row(a, u, t, g)[e] = O / L;
        } else {
            const int64_t ps = (pair + split) * t.gs + g;
            coherent_store(t.part_o + ps * dv + e, O);
            if (e == 0) {
                coherent_store(t.part_ml + ps * 2 + 0, M);
                coherent_store(t.part_ml + ps * 2 + 1, L);
            }
        }
    }
}

__device__ __forceinline__ int* pair_counter(const DecodeArgs& a, const DecodeUnit& u, const Tile& t) {
    return t.counters + (int64_t)u.qi * a.n_kv + u.kvh;
}

// Counts one finished split of u's pair; returns the count before it.  The
// split's partial must be complete (stored and waited for by every wave).
__device__ __forceinline__ int count_split(const DecodeArgs& a, const DecodeUnit& u, const Tile& t) {
    return __hip_atomic_fetch_add(pair_counter(a, u, t), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last split of u's pair to finish: out = sum_s 2^(m_s - M) O_s / sum_s
// 2^(m_s - M) l_s over all partials of the pair, then the counter goes back
// to zero.  General form, for pairs with many pieces: each thread loads the
// (m, l) and O of up to kMergeChunk splits at once per element it owns and
// folds chunks together with a running max, as the online softmax does.
__device__ __forceinline__ void merge_pair_chunked(const DecodeArgs& a, const DecodeUnit& u, const Tile& t) {
    const int tid = threadIdx.x;
    const int G = t.G;
    const int dv = t.dv;
    const int nsplit = u.split_info >> 16;
    const int64_t pair = (int64_t)u.slot;
    const int64_t stride = (int64_t)t.gs * dv;
    for (int idx = tid; idx < G * dv; idx += kDecodeThreads) {
        const int g = idx / dv;
        const int e = idx - g * dv;
        const float* po = t.part_o + (pair * t.gs + g) * dv + e;
        const float* pml = t.part_ml + (pair * t.gs + g) * 2;
        float M = -INFINITY, L = 0.f, O = 0.f;
        for (int s0 = 0; s0 < nsplit; s0 += kMergeChunk) {
            float ms[kMergeChunk], ls[kMergeChunk], os[kMergeChunk];
#pragma unroll
            for (int i = 0; i < kMergeChunk; ++i) {
                const bool in = s0 + i < nsplit;
                const int s = in ? s0 + i : s0;
                ms[i] = coherent_load(pml + (int64_t)s * t.gs * 2 + 0);
                ls[i] = coherent_load(pml + (int64_t)s * t.gs * 2 + 1);
                os[i] = coherent_load(po + s * stride);
                if (!in) ms[i] = -INFINITY;
            }
            float Mc = M;
#pragma unroll
            for (int i = 0; i < kMergeChunk; ++i) Mc = fmaxf(Mc, ms[i]);
            const float r = fast_exp2(M - Mc);  // 0 on the first chunk (M = -inf)
            L *= r;
            O *= r;
#pragma unroll
            for (int i = 0; i < kMergeChunk; ++i) {
                const float f = ms[i] == -INFINITY ? 0.f : fast_exp2(ms[i] - Mc);
                L = fmaf(ls[i], f, L);
                O = fmaf(os[i], f, O);
            }
            M = Mc;
        }
        out_row(a, u, t, g)[e] = O / L;
    }
    if (tid == 0) __hip_atomic_store(pair_counter(a, u, t), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The same merge for pairs with nsplit * G <= one (m, l) per thread.  Each
// coherent load pays a round trip to the memory side (about 1.3 us while HBM
// is busy), so the loads are issued together: the pieces' (m, l), one pair per
// thread, staged in LDS, and at the same time every out element this thread
// owns (kIdx of them) for kChunk pieces.  Thread g then forms head g's
// weights and sum once, and the weights go back through LDS.  A pair of up to
// kChunk pieces merges in one round trip, against one per owned element and
// chunk in the general form.
// Which form merges a pair depends on timing (the general one inside a
// workgroup's unit loop, this one after its last unit), so this form repeats
// the general form's arithmetic exactly: per group of kMergeChunk pieces the
// running max, the rescale of the sums by 2^(M - M_chunk), and the weights
// 2^(m_s - M_chunk), with every product and sum in the same order.  Results
// are then bit for bit the same whichever form runs.  `scr` is LDS the caller
// no longer reads, with room for 2 * nsplit * G + (nchunks + 1) * G floats.
template <int kIdx, int kLoads>
__device__ __forceinline__ void merge_pair_wide(const DecodeArgs& a, const DecodeUnit& u, const Tile& t, float* scr) {
    constexpr int kChunk = kLoads / kIdx;  // out loads in flight per thread: kIdx * kChunk
    const int tid = threadIdx.x;
    const int G = t.G;
    const int dv = t.dv;
    const int nsplit = u.split_info >> 16;
    const int n_ml = nsplit * G;
    const int64_t piece = (int64_t)t.gs * dv;  // floats per piece in part_o
    const float* po = t.part_o + (int64_t)u.slot * piece;
    const float* pml = t.part_ml + (int64_t)u.slot * t.gs * 2;
    const int nchunks = (nsplit + kMergeChunk - 1) / kMergeChunk;
    float* sm = scr;           // [s * G + g]: m, then the weight 2^(m - M_chunk)
    float* sl = scr + n_ml;    // [s * G + g]: l
    float* sinv = sl + n_ml;   // [g]: the sum over pieces (the divisor)
    float* sr = sinv + G;      // [c * G + g]: the rescale 2^(M - M_chunk) at chunk c

    float mt = -INFINITY, lt = 0.f;
    if (tid < n_ml) {
        const int s = tid / G;
        const int g = tid - s * G;
        mt = coherent_load(pml + ((int64_t)s * t.gs + g) * 2);
        lt = coherent_load(pml + ((int64_t)s * t.gs + g) * 2 + 1);
    }
    // Piece bases are wave-uniform and the lane's offset is one unsigned
    // index, so the loads take a scalar base and a 32-bit lane offset.
    float os[kIdx][kChunk];
    const unsigned lane_idx = (unsigned)tid;
    auto load_chunk = [&](int s0) {
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const float* pb = po + (int64_t)min(s0 + i, nsplit - 1) * piece;
#pragma unroll
            for (int k = 0; k < kIdx; ++k) {
                const unsigned idx = lane_idx + (unsigned)(k * kDecodeThreads);
                os[k][i] = (idx < (unsigned)(G * dv) && s0 + i < nsplit) ? coherent_load(pb + idx) : 0.f;
            }
        }
    };
    load_chunk(0);
    if (tid < n_ml) {
        sm[tid] = mt;
        sl[tid] = lt;
    }
    __syncthreads();
    if (tid < G) {
        // merge_pair_chunked's recurrence for head `tid`.
        float M = -INFINITY, L = 0.f;
        for (int c = 0; c < nchunks; ++c) {
            const int s1 = min(nsplit, (c + 1) * kMergeChunk);
            float Mc = M;
            for (int s = c * kMergeChunk; s < s1; ++s) Mc = fmaxf(Mc, sm[s * G + tid]);
            const float r = fast_exp2(M - Mc);  // 0 on the first chunk (M = -inf)
            sr[c * G + tid] = r;
            L *= r;
            for (int s = c * kMergeChunk; s < s1; ++s) {
                const float m = sm[s * G + tid];
                const float f = m == -INFINITY ? 0.f : fast_exp2(m - Mc);
                sm[s * G + tid] = f;
                L = fmaf(sl[s * G + tid], f, L);
            }
            M = Mc;
        }
        sinv[tid] = L;
    }
    __syncthreads();
    float O[kIdx];
#pragma unroll
    for (int k = 0; k < kIdx; ++k) O[k] = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += kChunk) {
        if (s0 > 0) load_chunk(s0);
#pragma unroll
        for (int k = 0; k < kIdx; ++k) {
            const int g = min(G - 1, (tid + k * kDecodeThreads) / dv);
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                const int s = s0 + i;
                if (s < nsplit) {
                    if (s % kMergeChunk == 0) O[k] *= sr[(s / kMergeChunk) * G + g];
                    O[k] = fmaf(os[k][i], sm[s * G + g], O[k]);
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kIdx; ++k) {
        const int idx = tid + k * kDecodeThreads;
        if (idx < G * dv) {
            const int g = idx / dv;
            out_row(a, u, t, g)[idx - g * dv] = O[k] / sinv[g];
        }
    }
    if (tid == 0) __hip_atomic_store(pair_counter(a, u, t), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge entry: the wide form when the pair's (m, l) fit one per thread and
// the LDS scratch, else the general one.  Called by every thread of the
// workgroup (the condition is workgroup-uniform); the epilogue's LDS is
// reused as scratch once all threads are past their reads of it.  kLoads is
// the out loads a thread keeps in flight; 0 keeps the general form, for call
// sites where the next unit's pages already hold most registers (the wide
// form spills there).
template <int D, int GMAX, int kLoads = 32>
__device__ __forceinline__ void merge_pair(const DecodeArgs& a, const DecodeUnit& u, const Tile& t,
                                           EpilogueLds<D, GMAX>& sh) {
    const int nsplit = u.split_info >> 16;
    const int n_ml = nsplit * t.G;
    const int n_scr = 2 * n_ml + ((nsplit + kMergeChunk - 1) / kMergeChunk + 1) * t.G;
    constexpr int kScratch = kDecodeWaves * GMAX * D;
    const int n_out = t.G * t.dv;
    if (kLoads > 0 && n_ml <= kDecodeThreads && n_scr <= kScratch && n_out <= 8 * kDecodeThreads) {
        __syncthreads();
        if (n_out <= 4 * kDecodeThreads)
            merge_pair_wide<4, (kLoads > 0 ? kLoads : 4)>(a, u, t, &sh.o[0][0][0]);
        else
            merge_pair_wide<8, (kLoads > 0 ? kLoads : 8)>(a, u, t, &sh.o[0][0][0]);
    } else {
        merge_pair_chunked(a, u, t);
    }
}

// publish_unit, then for a split piece the counter protocol on the spot:
// wait for the partial, count it, and merge the pair if it was the last one.
template <int D, int GMAX>
__device__ __forceinline__ void finish_unit(const DecodeArgs& a, const DecodeUnit& u, const Tile& t,
                                            EpilogueLds<D, GMAX>& sh) {
    publish_unit<D, GMAX>(a, u, t, sh);
    const int nsplit = u.split_info >> 16;
    if (nsplit == 1) return;
    wait_vm_complete();
    __syncthreads();
    if (threadIdx.x == 0) sh.last = (count_split(a, u, t) == nsplit - 1);
    __syncthreads();
    if (sh.last) merge_pair<D, GMAX>(a, u, t, sh);
}

}  // namespace gsp
