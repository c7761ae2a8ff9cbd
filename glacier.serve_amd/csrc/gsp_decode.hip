// DPP (VALU) decode kernel of the paged-attention step, written for gfx950
// (CDNA4, wave64).
//
// It computes PagedAttentionKernel.ComputeAttention
// (PagedAttentionKernel.cs:17-372) for every query token of a packed step:
//     s_t = dot(q_h, K[page(t), layer, hKv, slot(t)]) * attnScale   (:55-67)
//     p   = softmax(s[0 .. total))                                  (:70)
//     out = sum_t p_t V[page(t), layer, hKv, slot(t)]              (:73-370)
// with hKv = h / (nHeads / nHeadsKv) (:44,50).  The reference materialises the
// scores and makes three passes per query head; here one workgroup owns a
// (query token, KV head, page range) unit, reads each K/V page once for all G
// query heads of the GQA group, and keeps an online softmax (Milakov &
// Gimelshein 2018) in log2 units.
//
// Lane layout inside a wave: 16 lanes per token ("row"), 4 tokens per
// row-step, 4 row-steps per 16-token page.  Lane `sl` of a row holds
// head_dim/16 elements of the token: chunk c, element j sits at
// c * 16 * VEC + sl * VEC + j, so one load instruction of a row covers a
// contiguous 16*VEC-element stretch of the token (16-byte loads for fp32 and
// for fp16 at head_dim 128).  QK dot products are reduced across the 16 lanes
// of a row with DPP row rotations; the page maximum is reduced across the four
// rows with lane shuffles.  Each wave walks every kDecodeWaves-th page of the
// unit; the four waves merge through LDS and split units merge in the
// epilogue (gsp_epilogue.h).  The matrix-core kernel is the default; this one
// is kept for explicit selection and as an independent second implementation.
#include "gsp_epilogue.h"

namespace gsp {
namespace {

template <typename KT, int VEC>
struct VecOf;
template <>
struct VecOf<float, 4> {
    typedef float T __attribute__((ext_vector_type(4)));
};
template <>
struct VecOf<_Float16, 8> {
    typedef _Float16 T __attribute__((ext_vector_type(8)));
};
template <>
struct VecOf<_Float16, 4> {
    typedef _Float16 T __attribute__((ext_vector_type(4)));
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row, result in every lane of the row
// (row_ror:8, 4, 2, 1).
__device__ __forceinline__ float row_allsum16(float x) {
    x += dpp<0x128>(x);
    x += dpp<0x124>(x);
    x += dpp<0x122>(x);
    x += dpp<0x121>(x);
    return x;
}

template <int D, typename KT, int G>
__device__ __forceinline__ void decode_unit(const DecodeArgs& a, const DecodeUnit& u, EpilogueLds<D, G>& sh) {
    constexpr int S = D / 16;                                          // elements per lane
    constexpr int VEC = (sizeof(KT) == 4) ? 4 : (S >= 8 ? 8 : 4);      // elements per load
    constexpr int NCH = S / VEC;                                       // loads per token row
    constexpr int CH = 16 * VEC;                                       // distance between chunks
    typedef typename VecOf<KT, VEC>::T VT;

    const int kvh = u.kvh;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int trow = lane >> 4;
    const int sl = lane & 15;
    const int h0 = kvh * G;
    const int lane_off = sl * VEC;

    float q[G][S];
    {
        const float* qb = a.q + ((int64_t)u.qi * a.n_heads + h0) * D;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int j = 0; j < VEC; ++j) q[g][c * VEC + j] = qb[g * D + c * CH + lane_off + j];
    }

    float o[G][S];
    float m[G];
    float l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < S; ++e) o[g][e] = 0.f;
    }

    const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + kvh * a.head_stride;
    const KT* vbase = static_cast<const KT*>(a.v_pool) + a.layer_offset + kvh * a.head_stride;
    const float scale = a.scale_log2;

    for (int p = u.page_begin + wave; p < u.page_end; p += kDecodeWaves) {
#pragma clang fp contract(off)  // the max and the exponents see the same rounded scores
        const int64_t blk = a.bt_ids[u.bt_base + p];
        const KT* kp = kbase + blk * a.block_stride + lane_off;
        const KT* vp = vbase + blk * a.block_stride + lane_off;
        const int ntok = min(kBlockSize, u.ctx - p * kBlockSize);

        float k[4][S];
        float v[4][S];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = r * 4 + trow;
            if (t < ntok) {
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const VT kx = *reinterpret_cast<const VT*>(kp + t * D + c * CH);
                    const VT vx = *reinterpret_cast<const VT*>(vp + t * D + c * CH);
#pragma unroll
                    for (int j = 0; j < VEC; ++j) {
                        k[r][c * VEC + j] = static_cast<float>(kx[j]);
                        v[r][c * VEC + j] = static_cast<float>(vx[j]);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < S; ++e) {
                    k[r][e] = 0.f;
                    v[r][e] = 0.f;
                }
            }
        }

        float s[4][G];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool valid = (r * 4 + trow) < ntok;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float acc = 0.f;
#pragma unroll
                for (int e = 0; e < S; ++e) acc = fmaf(q[g][e], k[r][e], acc);
                acc = row_allsum16(acc);
                s[r][g] = valid ? acc * scale : -INFINITY;
            }
        }

#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mp = fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g]));
            mp = fmaxf(mp, __shfl_xor(mp, 16));
            mp = fmaxf(mp, __shfl_xor(mp, 32));
            if (mp > m[g]) {  // uniform across the wave: rescale only when the max grows
                const float alpha = fast_exp2(m[g] - mp);
                m[g] = mp;
                l[g] *= alpha;
#pragma unroll
                for (int e = 0; e < S; ++e) o[g][e] *= alpha;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = fast_exp2(s[r][g] - m[g]);
                l[g] += pr;
#pragma unroll
                for (int e = 0; e < S; ++e) o[g][e] = fmaf(pr, v[r][e], o[g][e]);
            }
        }
    }

    // Sum the four token rows of the wave; m is already uniform.
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l[g] += __shfl_xor(l[g], 16);
        l[g] += __shfl_xor(l[g], 32);
#pragma unroll
        for (int e = 0; e < S; ++e) {
            o[g][e] += __shfl_xor(o[g][e], 16);
            o[g][e] += __shfl_xor(o[g][e], 32);
        }
    }
    if (trow == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int j = 0; j < VEC; ++j) sh.o[wave][g][c * CH + lane_off + j] = o[g][c * VEC + j];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            sh.m[wave][g] = m[g];
            sh.l[wave][g] = l[g];
        }
    }
    __syncthreads();
    Tile t;  // the whole group (this kernel serves groups up to 8), full-width rows
    t.G = G;
    t.hoff = 0;
    t.gs = G;
    t.dv = D;
    t.part_o = a.part_o;
    t.part_ml = a.part_ml;
    t.counters = a.counters;
    finish_unit<D, G>(a, u, t, sh);
}

// One workgroup per bin; the bin's units run back to back.
template <int D, typename KT, int G>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(DecodeArgs a) {
    __shared__ EpilogueLds<D, G> sh;
    const int rb = a.bin_rest[blockIdx.x];
    const int re = a.bin_rest[blockIdx.x + 1];
    for (int k = rb - 1; k < re; ++k) {  // k = rb - 1: the bin's first unit, at index blockIdx.x
        decode_unit<D, KT, G>(a, a.units[k < rb ? (int)blockIdx.x : k], sh);
        __syncthreads();  // the epilogue LDS is reused by the next unit
    }
}

template <int D, typename KT, int G>
hipError_t launch_one(int num_bins, const DecodeArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL((paged_decode_kernel<D, KT, G>), dim3(num_bins), dim3(kDecodeThreads), 0, stream, a);
    return hipGetLastError();
}

template <int D, typename KT>
hipError_t launch_group(int group, int num_bins, const DecodeArgs& a, hipStream_t stream) {
    switch (group) {
        case 1: return launch_one<D, KT, 1>(num_bins, a, stream);
        case 2: return launch_one<D, KT, 2>(num_bins, a, stream);
        case 3: return launch_one<D, KT, 3>(num_bins, a, stream);
        case 4: return launch_one<D, KT, 4>(num_bins, a, stream);
        case 5: return launch_one<D, KT, 5>(num_bins, a, stream);
        case 6: return launch_one<D, KT, 6>(num_bins, a, stream);
        case 7: return launch_one<D, KT, 7>(num_bins, a, stream);
        case 8: return launch_one<D, KT, 8>(num_bins, a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_decode(int head_dim, int kv_f16, int num_bins, const DecodeArgs& a, hipStream_t stream) {
    if (num_bins <= 0) return hipSuccess;
    const int group = a.group;
    if (head_dim == 128)
        return kv_f16 ? launch_group<128, _Float16>(group, num_bins, a, stream)
                      : launch_group<128, float>(group, num_bins, a, stream);
    if (head_dim == 64)
        return kv_f16 ? launch_group<64, _Float16>(group, num_bins, a, stream)
                      : launch_group<64, float>(group, num_bins, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace gsp
