// Matrix-core (MFMA) kernel for chunked-prefill rows of the paged-attention
// step, gfx950.
//
// A prefill row stores its whole chunk first, then query token i attends to
// min(TokenCount, pos + i + 1) tokens (PagedTransformerRunner.cs:425-474,
// PagedAttentionKernel.cs:41).  Its queries share every K/V page of the prefix,
// so the work is a dense causal contraction; one workgroup owns a tile of 16
// consecutive query tokens of one row and one KV head, for all G <= 8 query
// heads of the GQA group, and walks the row's pages in order:
//
//   per page (16 keys, staged once in LDS and shared by the group's heads):
//     S^T[key][token] = K_page . Q_head^T   v_mfma_f32_16x16x4f32 (M = keys, N = tokens)
//     O_head[token][e] += P . V_page          v_mfma_f32_16x16x4f32 (M = tokens, K = keys)
//
// Row-tile T of the workgroup is query head kvh*G + T over the 16 tokens; wave
// w owns tiles w and w + 4.  The operand layouts are those of the decode
// kernel with "head" replaced by "query token", so each lane holds the scores
// of one token for four keys and the online softmax costs four exp2 per lane
// per page.  The causal limit is per row (token); padding rows past the
// tile's tokens keep finite scores and are never written.  Pages are staged
// through two LDS buffers (register-prefetched one page ahead) with one
// barrier per page.  The roofline of these rows is FP32 matrix throughput.
#include "gsp_epilogue.h"

namespace gsp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kPrefillTiles = kPrefillHeads / kDecodeWaves;  // row tiles (query heads) per wave
static_assert(kPrefillTileTokens == kBlockSize, "the tile's token and key dimensions are both 16");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t prefill_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

template <typename KT>
__device__ __forceinline__ f4 pload4(__amdgpu_buffer_rsrc_t r, int off);

template <>
__device__ __forceinline__ f4 pload4<float>(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4, 0, 0));
}

template <>
__device__ __forceinline__ f4 pload4<_Float16>(__amdgpu_buffer_rsrc_t r, int off) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 raw = __builtin_amdgcn_raw_buffer_load_b64(r, off * 2, 0, 0);
    const h4 h = __builtin_bit_cast(h4, raw);
    return f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

template <int D>
struct PrefillLds {
    static constexpr int kRow = D + 4;  // padded row: 16-byte skew between keys
    float k[2][kBlockSize * kRow];
    float v[2][kBlockSize * kRow];
};

// Each of the 256 threads moves (16 * D / 4) / 256 four-element chunks of K and of V.
template <int D>
struct StageRegs {
    f4 k[(kBlockSize * D / 4) / kDecodeThreads];
    f4 v[(kBlockSize * D / 4) / kDecodeThreads];
};

template <int D, typename KT>
__device__ __forceinline__ void stage_load(StageRegs<D>& sr, const KT* kpage, const KT* vpage, int ntok) {
    constexpr int NC = (kBlockSize * D / 4) / kDecodeThreads;
    const int bytes = ntok * D * (int)sizeof(KT);
    const __amdgpu_buffer_rsrc_t rk = prefill_rsrc(kpage, bytes);
    const __amdgpu_buffer_rsrc_t rv = prefill_rsrc(vpage, bytes);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = threadIdx.x + i * kDecodeThreads;  // chunk: key c / (D/4), elements 4 * (c % (D/4))
        sr.k[i] = pload4<KT>(rk, 4 * c);
        sr.v[i] = pload4<KT>(rv, 4 * c);
    }
}

template <int D>
__device__ __forceinline__ void stage_store(const StageRegs<D>& sr, float* lk, float* lv) {
    constexpr int NC = (kBlockSize * D / 4) / kDecodeThreads;
    constexpr int kRow = PrefillLds<D>::kRow;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = threadIdx.x + i * kDecodeThreads;
        const int key = c / (D / 4);
        const int col = 4 * (c % (D / 4));
        *reinterpret_cast<f4*>(lk + key * kRow + col) = sr.k[i];
        *reinterpret_cast<f4*>(lv + key * kRow + col) = sr.v[i];
    }
}

template <int D, typename KT>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_prefill_mfma_kernel(PrefillArgs a) {
    constexpr int kRow = PrefillLds<D>::kRow;
    __shared__ PrefillLds<D> sh;

    const PrefillTile t = a.tiles[blockIdx.x];
    const int hc = blockIdx.y * kPrefillHeads;  // first head of this workgroup within the group
    const int G = min(kPrefillHeads, a.group - hc);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;  // query token of the tile (B / result column)
    const int g = lane >> 4;
    const int h0 = t.kvh * a.group + hc;
    // Tokens this lane's row attends to; padding rows past the tile get the
    // whole page range so their scores stay finite.
    const bool row_live = n < t.ntok;
    const int row_ctx = row_live ? min(t.token_count, t.pos0 + n + 1) : 0x7fffffff;
    const float scale = a.scale_log2;

    // Q^T operands and accumulators of this wave's tiles (tile T = head T).
    f4 q[kPrefillTiles][D / 16];
    f4 o[kPrefillTiles][D / 16];
    float m[kPrefillTiles], l[kPrefillTiles];
#pragma unroll
    for (int s = 0; s < kPrefillTiles; ++s) {
        const int T = wave + 4 * s;
        const bool live = T < G && row_live;
        const float* qrow = a.q + ((int64_t)(t.qi0 + (row_live ? n : 0)) * a.n_heads + h0 + (T < G ? T : 0)) * D;
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
            const f4 x = *reinterpret_cast<const f4*>(qrow + 16 * j + 4 * g);
            q[s][j] = live ? x : f4{0.f, 0.f, 0.f, 0.f};
            o[s][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
        m[s] = -INFINITY;
        l[s] = 0.f;
    }

    const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)t.kvh * a.head_stride;
    const KT* vbase = static_cast<const KT*>(a.v_pool) + a.layer_offset + (int64_t)t.kvh * a.head_stride;
    const int32_t* bt = a.bt_ids + t.bt_base;
    const int ctx_last = min(t.token_count, t.pos0 + t.ntok);

    StageRegs<D> sr;
    {
        const int64_t blk = bt[0];
        stage_load<D, KT>(sr, kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                          min(kBlockSize, ctx_last));
        stage_store<D>(sr, sh.k[0], sh.v[0]);
    }
    __syncthreads();

    for (int p = 0; p < t.pages; ++p) {
        const int buf = p & 1;
        if (p + 1 < t.pages) {
            const int64_t blk = bt[p + 1];
            stage_load<D, KT>(sr, kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                              min(kBlockSize, ctx_last - (p + 1) * kBlockSize));
        }
        // K operand: K[key n][16j + 4g ..]; V operand: V[key 4g + kk][64c + 4n ..].
        const float* lk = sh.k[buf];
        const float* lv = sh.v[buf];
        f4 kop[D / 16];
#pragma unroll
        for (int j = 0; j < D / 16; ++j) kop[j] = *reinterpret_cast<const f4*>(lk + n * kRow + 16 * j + 4 * g);
        f4 vop[4][D / 64];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int c = 0; c < D / 64; ++c)
                vop[kk][c] = *reinterpret_cast<const f4*>(lv + (4 * g + kk) * kRow + 64 * c + 4 * n);

        const int key0 = p * kBlockSize + 4 * g;
        const bool diag = (p + 1) * kBlockSize > min(t.pos0 + 1, t.token_count);  // some row may stop here
#pragma unroll
        for (int s = 0; s < kPrefillTiles; ++s) {
            if (wave + 4 * s >= G) continue;  // uniform per wave
            f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < D / 16; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (j & 1)
                        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kop[j][i], q[s][j][i], s1, 0, 0, 0);
                    else
                        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kop[j][i], q[s][j][i], s0, 0, 0, 0);
                }
            f4 sc = (s0 + s1) * scale;  // lane: S[token n][keys key0 .. key0 + 3]
            if (diag) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (key0 + r >= row_ctx) sc[r] = -INFINITY;
            }
            float mp = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            mp = fmaxf(mp, __shfl_xor(mp, 16));
            mp = fmaxf(mp, __shfl_xor(mp, 32));
            const float mn = fmaxf(m[s], mp);  // finite: page 0 holds key 0 for every row
            const float alpha = fast_exp2(m[s] - mn);
            m[s] = mn;
            f4 pr;
#pragma unroll
            for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(sc[r] - mn);
            l[s] = l[s] * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
            if (__any(alpha != 1.0f)) {
                const int src = 4 * g;
                f4 ar;
#pragma unroll
                for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, src + r);
#pragma unroll
                for (int b = 0; b < D / 16; ++b) o[s][b] *= ar;
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int c = 0; c < D / 64; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][4 * c + i] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(pr[kk], vop[kk][c][i], o[s][4 * c + i], 0, 0, 0);
        }
        if (p + 1 < t.pages) stage_store<D>(sr, sh.k[buf ^ 1], sh.v[buf ^ 1]);
        __syncthreads();
    }

    // O rows are tokens 4g + r of head T; l of token n lives in lanes n (+16k).
#pragma unroll
    for (int s = 0; s < kPrefillTiles; ++s) {
        const int T = wave + 4 * s;
        if (T >= G) continue;
        float ls = l[s];
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        f4 inv;
#pragma unroll
        for (int r = 0; r < 4; ++r) inv[r] = 1.0f / __shfl(ls, 4 * g + r);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 4 * g + r;
            if (tok < t.ntok) {
                float* orow = a.out + ((int64_t)(t.qi0 + tok) * a.n_heads + h0 + T) * D;
#pragma unroll
                for (int c = 0; c < D / 64; ++c) {
                    f4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = o[s][4 * c + i][r] * inv[r];
                    *reinterpret_cast<f4*>(orow + 64 * c + 4 * n) = v;
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_prefill_mfma(int head_dim, int kv_f16, int num_tiles, const PrefillArgs& a, hipStream_t stream) {
    if (num_tiles <= 0) return hipSuccess;
    if (a.group < 1) return hipErrorInvalidValue;
    dim3 grid(num_tiles, (a.group + kPrefillHeads - 1) / kPrefillHeads);
    if (head_dim == 128) {
        if (kv_f16)
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<128, _Float16>), grid, dim3(kDecodeThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<128, float>), grid, dim3(kDecodeThreads), 0, stream, a);
    } else if (head_dim == 64) {
        if (kv_f16)
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<64, _Float16>), grid, dim3(kDecodeThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<64, float>), grid, dim3(kDecodeThreads), 0, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gsp
