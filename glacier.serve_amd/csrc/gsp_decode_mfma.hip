// Matrix-core (MFMA) decode kernel of the paged-attention step, gfx950.
//
// Same contract as the DPP decode kernel (PagedAttentionKernel.cs:17-372 over
// every query token of a packed step), but the GQA group turns each 16-token
// page into two small dense contractions that run on the matrix cores:
//
//   S^T[token][head] = K_page[16 x d] . (Q_group * scale * log2 e)^T   (v_mfma_f32_16x16x4f32, M = tokens, N = heads)
//   O[head][e]      += P[16 heads x 16 tokens] . V_page[16 x d]          (v_mfma_f32_16x16x4f32, M = heads, K = tokens)
//
// Heads of the group beyond G are zero padding (G <= 16).  MFMA operand
// layouts (lane l, n = l % 16, g = l / 16):
//   QK step kk = 4j + i uses d = 16j + 4g + i:  A = K[token n][d],  B = Q[head n][d]
//   result: lane holds S[head n][token 4g + r], r = 0..3
//   PV step kk uses token 4g + kk:  A = P[head n][token 4g + kk] (the lane's own r = kk),
//   B = V[token 4g + kk][e], e = 64c + 4n + i for output block 4c + i
//   result: lane holds O[head 4g + r][e].
// So each lane reads 16-byte pieces of K rows and V rows straight into MFMA
// operands; the softmax needs one max-reduction across the four lane groups
// per page and four exp2 per lane.  Page loads are raw buffer loads whose
// descriptor covers only the page's valid tokens: slots past the context read
// as zero in hardware (no fetch, no NaN from stale slots reaches P.V).  Each
// wave streams every kDecodeWaves-th page of its unit with the next page's
// loads in flight while the current one is computed; the four waves merge
// through LDS and split units merge in the epilogue (gsp_epilogue.h).
#include "gsp_epilogue.h"

namespace gsp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* base, int bytes) {
    // Raw buffer (stride 0) of `bytes` bytes; offsets at or past the end read 0.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// 4 consecutive elements of a K/V row at element offset `off`, as fp32.
template <typename KT>
__device__ __forceinline__ f4 load4(__amdgpu_buffer_rsrc_t r, int off);

template <>
__device__ __forceinline__ f4 load4<float>(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4, 0, 0));
}

template <>
__device__ __forceinline__ f4 load4<_Float16>(__amdgpu_buffer_rsrc_t r, int off) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 raw = __builtin_amdgcn_raw_buffer_load_b64(r, off * 2, 0, 0);
    const h4 h = __builtin_bit_cast(h4, raw);
    return f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

template <int D>
struct PageRegs {
    f4 k[D / 16];          // K[token n][16j + 4g .. +3]
    f4 v[4][D / 64];       // V[token 4g + kk][64c + 4n .. +3]
};

template <int D, typename KT>
__device__ __forceinline__ void load_page(PageRegs<D>& pr, const KT* kpage, const KT* vpage, int ntok, int n,
                                          int g) {
    const int bytes = ntok * D * (int)sizeof(KT);
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(kpage, bytes);
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(vpage, bytes);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) pr.k[j] = load4<KT>(rk, n * D + 16 * j + 4 * g);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int c = 0; c < D / 64; ++c) pr.v[kk][c] = load4<KT>(rv, (4 * g + kk) * D + 64 * c + 4 * n);
}

template <int D>
struct WaveState {
    f4 o[D / 16];  // O[head 4g + r][64c + 4n + i] for block b = 4c + i
    float m;       // running max (log2 units) of head n
    float l;       // partial sum of head n over this lane's tokens
};

template <int D>
__device__ __forceinline__ void compute_page(WaveState<D>& st, const PageRegs<D>& pr, const f4 (&q)[D / 16],
                                             float scale, int ntok, int g) {
    // S^T = K . Q^T: 32 (d = 128) or 16 (d = 64) rank-4 steps, two accumulation chains.
    f4 s0 = {0.f, 0.f, 0.f, 0.f};
    f4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (j & 1)
                s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(pr.k[j][i], q[j][i], s1, 0, 0, 0);
            else
                s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(pr.k[j][i], q[j][i], s0, 0, 0, 0);
        }
    }
    f4 s = (s0 + s1) * scale;  // lane: S[head n][token 4g + r] in log2 units
    if (ntok < kBlockSize) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r >= ntok) s[r] = -INFINITY;
    }
    float mp = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mp = fmaxf(mp, __shfl_xor(mp, 16));
    mp = fmaxf(mp, __shfl_xor(mp, 32));
    const float mn = fmaxf(st.m, mp);
    const float alpha = fast_exp2(st.m - mn);  // 0 on the first page (m = -inf)
    st.m = mn;
    f4 p;
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(s[r] - mn);
    st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    // O rows are heads 4g + r; their alphas live in lanes 4g + r.
    if (__any(alpha != 1.0f)) {
        const int lane = threadIdx.x & 63;
        const int src = 4 * (lane >> 4);
        f4 ar;
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, src + r);
#pragma unroll
        for (int b = 0; b < D / 16; ++b) st.o[b] *= ar;
    }
    // O += P . V: 4 token steps x D/16 output blocks.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int c = 0; c < D / 64; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st.o[4 * c + i] =
                    __builtin_amdgcn_mfma_f32_16x16x4f32(p[kk], pr.v[kk][c][i], st.o[4 * c + i], 0, 0, 0);
}

// Step metadata (unit records, bin offsets, block table) is read-only while
// the kernel runs.  Reading it through the constant address space lets the
// compiler use scalar loads even though the epilogue stores inside the bin
// loop: a vector load there would be followed by a full vmcnt(0) wait that
// also drains the page loads in flight.
typedef __attribute__((address_space(4))) const int32_t const_i32;

__device__ __forceinline__ int ld_meta(const int32_t* p) { return *(const_i32*)p; }

// The scalar fields of unit `ui`; first_blk is read separately (first_block).
__device__ __forceinline__ DecodeUnit read_unit(const DecodeArgs& a, int ui) {
    const int32_t* src = reinterpret_cast<const int32_t*>(a.units + ui);
    DecodeUnit u;
    u.qi = ld_meta(src + 0);
    u.bt_base = ld_meta(src + 1);
    u.page_begin = ld_meta(src + 2);
    u.page_end = ld_meta(src + 3);
    u.ctx = ld_meta(src + 4);
    u.kvh = ld_meta(src + 5);
    u.slot = ld_meta(src + 6);
    u.split_info = ld_meta(src + 7);
    return u;
}

// Q^T operand of a unit: q[j][i] = Q[kvh * G + n][16j + 4g + i]; padded heads
// are 0.  The scale (times log2 e) multiplies S after the MFMA, as the
// reference multiplies the finished dot (PagedAttentionKernel.cs:65).
template <int D>
__device__ __forceinline__ void load_q(f4 (&q)[D / 16], const DecodeArgs& a, const DecodeUnit& u, int G, int n,
                                       int g) {
    const bool live = n < G;
    const float* qrow = a.q + ((int64_t)u.qi * a.n_heads + u.kvh * G + (live ? n : 0)) * D;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        const f4 x = *reinterpret_cast<const f4*>(qrow + 16 * j + 4 * g);
        q[j] = live ? x : f4{0.f, 0.f, 0.f, 0.f};
    }
}

// The block id of this wave's first page of unit `ui` (page_begin + wave),
// which travels in the unit record so the first load needs no table lookup.
// It is read from the record in memory with wave-uniform indices: a local
// copy indexed by `wave` would live in per-lane memory and turn the page
// address divergent.
__device__ __forceinline__ int first_block(const DecodeArgs& a, int ui, int wave) {
    return ld_meta(reinterpret_cast<const int32_t*>(a.units + ui) + 8 + wave);
}

template <int D, typename KT>
__device__ __forceinline__ void load_first_page(PageRegs<D>& pr, const DecodeArgs& a, const DecodeUnit& u, int blk,
                                                int wave, int n, int g) {
    const int p = u.page_begin + wave;
    if (p < u.page_end) {
        const int64_t off = a.layer_offset + (int64_t)u.kvh * a.head_stride + (int64_t)blk * a.block_stride;
        load_page<D, KT>(pr, static_cast<const KT*>(a.k_pool) + off, static_cast<const KT*>(a.v_pool) + off,
                         min(kBlockSize, u.ctx - p * kBlockSize), n, g);
    }
}

// One workgroup per bin: unit blockIdx.x, then units [bin_rest[b], bin_rest[b + 1]),
// back to back.  Before a unit's epilogue (wave merge, partial publish, split
// merge) the next unit's Q and first pages are already requested, so the
// CU's load stream keeps going across unit boundaries.
template <int D, typename KT>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_decode_mfma_kernel(DecodeArgs a) {
    __shared__ EpilogueLds<D, kMaxGroupMfma> sh;

    const int G = a.group;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int g = lane >> 4;
    const float scale = a.scale_log2;
    const int first = blockIdx.x;

    f4 q[D / 16];
    PageRegs<D> ra, rb;
    {
        const DecodeUnit u0 = read_unit(a, first);
        const int blk0 = first_block(a, first, wave);
        load_q<D>(q, a, u0, G, n, g);
        load_first_page<D, KT>(ra, a, u0, blk0, wave, n, g);
    }
    const int rb0 = ld_meta(a.bin_rest + first);
    const int re = ld_meta(a.bin_rest + first + 1);

    // The unit record is re-read from memory in every iteration (wave-uniform
    // address), never carried across iterations, so every field stays scalar.
    for (int k = rb0 - 1; k < re; ++k) {
        const int ui = k < rb0 ? first : k;
        const DecodeUnit u = read_unit(a, ui);
        const bool has_next = k + 1 < re;
        // The next record is fetched now; its latency hides behind this unit.
        const DecodeUnit un = read_unit(a, has_next ? k + 1 : ui);
        const int blkn = first_block(a, has_next ? k + 1 : ui, wave);

        WaveState<D> st;
#pragma unroll
        for (int b = 0; b < D / 16; ++b) st.o[b] = f4{0.f, 0.f, 0.f, 0.f};
        st.m = -INFINITY;
        st.l = 0.f;

        const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)u.kvh * a.head_stride;
        const KT* vbase = static_cast<const KT*>(a.v_pool) + a.layer_offset + (int64_t)u.kvh * a.head_stride;
        const int32_t* bt = a.bt_ids + u.bt_base;

        // Two page buffers in flight: load page p + kDecodeWaves while computing page p.
        int p = u.page_begin + wave;
        while (p < u.page_end) {
            const int pn = p + kDecodeWaves;
            if (pn < u.page_end) {
                const int64_t blk = ld_meta(bt + pn);
                load_page<D, KT>(rb, kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                                 min(kBlockSize, u.ctx - pn * kBlockSize), n, g);
            }
            compute_page<D>(st, ra, q, scale, min(kBlockSize, u.ctx - p * kBlockSize), g);
            if (pn >= u.page_end) break;
            const int pnn = pn + kDecodeWaves;
            if (pnn < u.page_end) {
                const int64_t blk = ld_meta(bt + pnn);
                load_page<D, KT>(ra, kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                                 min(kBlockSize, u.ctx - pnn * kBlockSize), n, g);
            }
            compute_page<D>(st, rb, q, scale, min(kBlockSize, u.ctx - pn * kBlockSize), g);
            p = pnn;
        }

        // Both page buffers and q are free now: request the next unit's inputs.
        if (has_next) {
            load_q<D>(q, a, un, G, n, g);
            load_first_page<D, KT>(ra, a, un, blkn, wave, n, g);
        }

        // Per-head sums over the four lane groups; m is uniform per head already.
        st.l += __shfl_xor(st.l, 16);
        st.l += __shfl_xor(st.l, 32);
        if (g == 0 && n < G) {
            sh.m[wave][n] = st.m;
            sh.l[wave][n] = st.l;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            if (h < G) {
#pragma unroll
                for (int c = 0; c < D / 64; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) sh.o[wave][h][64 * c + 4 * n + i] = st.o[4 * c + i][r];
            }
        }
        __syncthreads();
        finish_unit<D, kMaxGroupMfma>(a, u, G, sh);
        __syncthreads();  // the epilogue LDS is reused by the next unit
    }
}

}  // namespace

hipError_t launch_decode_mfma(int head_dim, int kv_f16, int num_bins, const DecodeArgs& a, hipStream_t stream) {
    if (num_bins <= 0) return hipSuccess;
    dim3 grid(num_bins);
    if (head_dim == 128) {
        if (kv_f16)
            hipLaunchKernelGGL((paged_decode_mfma_kernel<128, _Float16>), grid, dim3(kDecodeThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((paged_decode_mfma_kernel<128, float>), grid, dim3(kDecodeThreads), 0, stream, a);
    } else if (head_dim == 64) {
        if (kv_f16)
            hipLaunchKernelGGL((paged_decode_mfma_kernel<64, _Float16>), grid, dim3(kDecodeThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((paged_decode_mfma_kernel<64, float>), grid, dim3(kDecodeThreads), 0, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gsp
