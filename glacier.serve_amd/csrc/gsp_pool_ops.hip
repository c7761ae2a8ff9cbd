// Device page operations on the KV pool (gfx950): the batched Store scatter,
// the same scatter with the rotary embedding applied on the way, and the
// copy-on-write page copy.  All are small HBM-bound copies.
#include "gsp_internal.h"
#include "../../include/glacier_paged.h"

namespace gsp {
namespace {

// PagedBlockPool.Store (PagedBlockPool.cs:151-161) for n tokens at once:
// token i, KV head h -> K/V[block_ids[i]][layer][h][slots[i]][:].  One
// workgroup per (token, head); fp32 -> fp16 rounds to nearest even.  A token
// with block id -1 has no slot and is skipped.  The first 256 elements of a
// head are loaded (two per thread) together with the block id and slot, so
// the usual head costs one memory round trip; wider heads loop on.
template <typename KT>
__global__ __launch_bounds__(128) void write_tokens_kernel(WriteTokensArgs a) {
    const int i = blockIdx.x;
    const int h = blockIdx.y;
    const float* ks = a.k + ((int64_t)i * a.n_kv + h) * a.head_dim;
    const float* vs = a.v + ((int64_t)i * a.n_kv + h) * a.v_head_dim;
    const int e0 = threadIdx.x, e1 = threadIdx.x + 128;
    const float k0 = e0 < a.head_dim ? ks[e0] : 0.f, k1 = e1 < a.head_dim ? ks[e1] : 0.f;
    const float v0 = e0 < a.v_head_dim ? vs[e0] : 0.f, v1 = e1 < a.v_head_dim ? vs[e1] : 0.f;
    const int64_t blk = a.block_ids[i];
    const int64_t slot = a.slots[i];
    if (blk < 0) return;
    KT* kd = static_cast<KT*>(a.k_pool) + blk * a.block_stride + a.layer_offset + h * a.head_stride + slot * a.head_dim;
    KT* vd = static_cast<KT*>(a.v_pool) + blk * a.v_block_stride + a.v_layer_offset + h * a.v_head_stride +
             slot * a.v_head_dim;
    if (e0 < a.head_dim) kd[e0] = static_cast<KT>(k0);
    if (e1 < a.head_dim) kd[e1] = static_cast<KT>(k1);
    if (e0 < a.v_head_dim) vd[e0] = static_cast<KT>(v0);
    if (e1 < a.v_head_dim) vd[e1] = static_cast<KT>(v1);
    for (int e = e0 + 256; e < a.head_dim; e += 128) kd[e] = static_cast<KT>(ks[e]);
    for (int e = e0 + 256; e < a.v_head_dim; e += 128) vd[e] = static_cast<KT>(vs[e]);
}

// Cosine and sine of pair j's angle at position `pos`, times the rotation's
// scale (shared by both RoPE kernels).  The angle, pos times the pair's rate
// (the table's, or freq_base^(-2j/rope_dim)), is formed and reduced to
// [-pi, pi] in fp64, so it stays exact at long positions; cosine and sine are
// fp32.  A scale of 1 leaves them exact.
__device__ inline void rope_angle(const RopeWriteArgs& a, double pos, int j, float* c, float* s) {
    const double rate = a.freq ? a.freq[j] : exp2(-(2.0 * j / a.rope_dim) * a.log2_base);
    const double ang = pos * rate;
    const double r = ang - 6.283185307179586 * rint(ang * 0.15915494309189535);
    float sn, cn;
    sincosf((float)r, &sn, &cn);
    *c = cn * a.mscale;
    *s = sn * a.mscale;
}

__device__ inline void rope_turn(float x0, float x1, float c, float s, float* y0, float* y1) {
    *y0 = x0 * c - x1 * s;
    *y1 = x0 * s + x1 * c;
}

// QuantKernels.RoPE then PagedBlockPool.Store for n tokens
// (PagedTransformerRunner.cs:253-267, 436-449, 619-634), one workgroup per
// token.  Pair j < rope_dim/2 of every head turns by its angle (Su et al.,
// RoFormer; rope_angle), taken once per token; dims from rope_dim on pass
// through.  Q heads are rotated in place, K heads are rotated into the pool
// slot and V is stored as is; fp16 pools round to nearest even.  A token with
// block id -1 has no slot: its Q is rotated, its K and V are not stored.
template <typename KT>
__global__ __launch_bounds__(256) void rope_write_kernel(RopeWriteArgs a) {
    __shared__ float cs[kRopeMaxHalf][2];
    const int i = blockIdx.x;
    const int d = a.head_dim;
    const int half = a.rope_dim >> 1;
    const double pos = (double)a.positions[i];
    for (int j = threadIdx.x; j < half; j += blockDim.x) rope_angle(a, pos, j, &cs[j][0], &cs[j][1]);
    __syncthreads();
    const bool stored = a.block_ids[i] >= 0;
    const int64_t dst = (int64_t)a.block_ids[i] * a.block_stride + a.layer_offset + (int64_t)a.slots[i] * d;
    const int dv = a.v_head_dim;
    const int64_t vdst = (int64_t)a.block_ids[i] * a.v_block_stride + a.v_layer_offset + (int64_t)a.slots[i] * dv;
    const bool pairs = a.style == GSP_ROPE_PAIRS;
    const int heads = a.n_heads + (stored ? a.n_kv : 0);
    for (int idx = threadIdx.x; idx < heads * half; idx += blockDim.x) {
        const int h = idx / half;
        const int j = idx - h * half;
        const int e0 = pairs ? 2 * j : j;
        const int e1 = pairs ? 2 * j + 1 : j + half;
        const float c = cs[j][0];
        const float s = cs[j][1];
        if (h < a.n_heads) {
            float* q = a.q + ((int64_t)i * a.n_heads + h) * d;
            const float x0 = q[e0], x1 = q[e1];
            q[e0] = x0 * c - x1 * s;
            q[e1] = x0 * s + x1 * c;
        } else {
            const int hk = h - a.n_heads;
            const float* k = a.k + ((int64_t)i * a.n_kv + hk) * d;
            KT* kd = static_cast<KT*>(a.k_pool) + dst + (int64_t)hk * a.head_stride;
            const float x0 = k[e0], x1 = k[e1];
            kd[e0] = static_cast<KT>(x0 * c - x1 * s);
            kd[e1] = static_cast<KT>(x0 * s + x1 * c);
        }
    }
    // K dims past rope_dim go to the pool as they are.
    const int tail = d - a.rope_dim;
    for (int idx = threadIdx.x; stored && idx < a.n_kv * tail; idx += blockDim.x) {
        const int hk = idx / tail;
        const int e = a.rope_dim + (idx - hk * tail);
        static_cast<KT*>(a.k_pool)[dst + (int64_t)hk * a.head_stride + e] =
            static_cast<KT>(a.k[((int64_t)i * a.n_kv + hk) * d + e]);
    }
    for (int idx = threadIdx.x; stored && idx < a.n_kv * dv; idx += blockDim.x) {
        const int hk = idx / dv;
        const int e = idx - hk * dv;
        static_cast<KT*>(a.v_pool)[vdst + (int64_t)hk * a.v_head_stride + e] =
            static_cast<KT>(a.v[((int64_t)i * a.n_kv + hk) * dv + e]);
    }
}

template <typename KT>
__device__ inline void store4(KT* p, const float4& x) {
    if constexpr (sizeof(KT) == 4) {
        *reinterpret_cast<float4*>(p) = x;
    } else {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 h = {(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
        *reinterpret_cast<h4*>(p) = h;
    }
}

// The same RoPE and Store with 16-byte accesses, for head_dim % 8 == 0,
// rope_dim % 8 == 0, v_head_dim % 4 == 0 and 16-byte aligned buffers.  A
// token's work is a list of items: per Q head and per K head, head_dim / 8
// items, the first rope_dim / 8 of four rotation pairs (two float4 of the
// head) and the rest of eight dims past rope_dim (two float4 passed through:
// nothing to do for Q, a copy into the pool for K), then per V head
// v_head_dim / 4 items of one float4.  Workgroup (token, y) takes items
// [256 y, 256 y + 256), one per thread.  The item list does not depend on the
// token's block id (a token with none skips its K and V stores at the end),
// so each thread issues its loads together with the token's position, block
// and slot, before the angle table is built: a workgroup costs about one
// memory round trip.
template <typename KT>
__global__ __launch_bounds__(256) void rope_write_vec_kernel(RopeWriteArgs a) {
    __shared__ float cs[kRopeMaxHalf][2];
    const int i = blockIdx.x;
    const int d = a.head_dim;
    const int half = a.rope_dim >> 1;
    const int rot_items = a.rope_dim >> 3;
    const int dv = a.v_head_dim;
    const int per_head = d >> 3;
    const int nq = a.n_heads * per_head;
    const int nk = a.n_kv * per_head;
    const int nv = a.n_kv * (dv >> 2);
    const int t = blockIdx.y * 256 + threadIdx.x;
    const bool pairs = a.style == GSP_ROPE_PAIRS;

    // Item geometry: the head's two float4 (or the V float4) and the first pair.
    int kind = 3;  // 0 Q, 1 K, 2 V, 3 none
    int h = 0, m = 0;
    if (t < nq) {
        kind = 0;
        h = t / per_head;
        m = t - h * per_head;
    } else if (t < nq + nk) {
        kind = 1;
        h = (t - nq) / per_head;
        m = (t - nq) - h * per_head;
    } else if (t < nq + nk + nv) {
        kind = 2;
        h = (t - nq - nk) / (dv >> 2);
        m = (t - nq - nk) - h * (dv >> 2);
    }
    // Rotation items: halves, elements 4m.. and half+4m.., pairs 4m..4m+3;
    // pairs, elements 8m.. and 8m+4.., pairs 4m..4m+3.  Items past rope_dim:
    // elements 8m..8m+7, which Q keeps and K copies.
    const bool turn = m < rot_items;
    if (kind == 0 && !turn) kind = 3;
    const int e0 = pairs || !turn ? 8 * m : 4 * m;
    const int e1 = pairs || !turn ? 8 * m + 4 : 4 * m + half;
    const float* src = kind == 0 ? a.q + ((int64_t)i * a.n_heads + h) * d
                     : kind == 1 ? a.k + ((int64_t)i * a.n_kv + h) * d
                                 : a.v + ((int64_t)i * a.n_kv + h) * dv;
    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
    if (kind == 0 || kind == 1) {
        x0 = *reinterpret_cast<const float4*>(src + e0);
        x1 = *reinterpret_cast<const float4*>(src + e1);
    } else if (kind == 2) {
        x0 = *reinterpret_cast<const float4*>(src + 4 * m);
    }

    const double pos = (double)a.positions[i];
    const int64_t blk = a.block_ids[i];
    const int64_t slot = a.slots[i];
    for (int j = threadIdx.x; j < half; j += 256) rope_angle(a, pos, j, &cs[j][0], &cs[j][1]);
    __syncthreads();

    if (kind == 3 || (kind != 0 && blk < 0)) return;
    if (kind == 2) {
        KT* vd = static_cast<KT*>(a.v_pool) + blk * a.v_block_stride + a.v_layer_offset +
                 (int64_t)h * a.v_head_stride + slot * dv;
        store4(vd + 4 * m, x0);
        return;
    }
    const int j0 = 4 * m;
    float4 y0 = x0, y1 = x1;
    if (!turn) {
        // K dims past rope_dim: stored as they are.
    } else if (pairs) {
        rope_turn(x0.x, x0.y, cs[j0][0], cs[j0][1], &y0.x, &y0.y);
        rope_turn(x0.z, x0.w, cs[j0 + 1][0], cs[j0 + 1][1], &y0.z, &y0.w);
        rope_turn(x1.x, x1.y, cs[j0 + 2][0], cs[j0 + 2][1], &y1.x, &y1.y);
        rope_turn(x1.z, x1.w, cs[j0 + 3][0], cs[j0 + 3][1], &y1.z, &y1.w);
    } else {
        rope_turn(x0.x, x1.x, cs[j0][0], cs[j0][1], &y0.x, &y1.x);
        rope_turn(x0.y, x1.y, cs[j0 + 1][0], cs[j0 + 1][1], &y0.y, &y1.y);
        rope_turn(x0.z, x1.z, cs[j0 + 2][0], cs[j0 + 2][1], &y0.z, &y1.z);
        rope_turn(x0.w, x1.w, cs[j0 + 3][0], cs[j0 + 3][1], &y0.w, &y1.w);
    }
    if (kind == 0) {
        float* q = a.q + ((int64_t)i * a.n_heads + h) * d;
        *reinterpret_cast<float4*>(q + e0) = y0;
        *reinterpret_cast<float4*>(q + e1) = y1;
    } else {
        KT* kd = static_cast<KT*>(a.k_pool) + blk * a.block_stride + a.layer_offset + (int64_t)h * a.head_stride +
                 slot * d;
        store4(kd + e0, y0);
        store4(kd + e1, y1);
    }
}

// PagedBlockPool.CopyBlockData (PagedBlockPool.cs:304-327): the first
// valid_tokens slots of every (layer, KV head) page of `src` go to `dst`.
template <typename KT>
__global__ __launch_bounds__(256) void copy_block_kernel(CopyBlockArgs a) {
    const int lh = blockIdx.x;  // layer * n_kv + head: pages are consecutive
    const int64_t nk = (int64_t)a.valid_tokens * a.head_dim;
    const int64_t nv = (int64_t)a.valid_tokens * a.v_head_dim;
    const KT* ks = static_cast<const KT*>(a.k_pool) + (int64_t)a.src * a.block_stride + (int64_t)lh * a.head_stride;
    const KT* vs = static_cast<const KT*>(a.v_pool) + (int64_t)a.src * a.v_block_stride + (int64_t)lh * a.v_head_stride;
    KT* kd = static_cast<KT*>(a.k_pool) + (int64_t)a.dst * a.block_stride + (int64_t)lh * a.head_stride;
    KT* vd = static_cast<KT*>(a.v_pool) + (int64_t)a.dst * a.v_block_stride + (int64_t)lh * a.v_head_stride;
    for (int64_t e = threadIdx.x; e < nk; e += blockDim.x) kd[e] = ks[e];
    for (int64_t e = threadIdx.x; e < nv; e += blockDim.x) vd[e] = vs[e];
}

// Sets n int32 words to `value`.  Used instead of hipMemsetAsync where a
// caller may capture the call into a graph.
__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, int64_t n, int32_t value) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = value;
}

// Copies the packed step from its pinned staging buffer into the step's
// device slot, n16 16-byte words.  The staging buffer is fine-grained host
// memory, which the GPU reads over the bus without caching it, so each load
// sees what the host wrote before the launch.  A kernel on the step's stream
// follows the previous step's kernel within a few microseconds, where a DMA
// copy between two kernels measured an 18-20 us gap per step.
__global__ __launch_bounds__(256) void upload_step_kernel(const uint4* src, uint4* dst, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

}  // namespace

hipError_t launch_upload_step(const void* src, void* dst, int64_t n16, hipStream_t stream) {
    if (n16 <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 1024);
    hipLaunchKernelGGL(upload_step_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const uint4*>(src),
                       static_cast<uint4*>(dst), n16);
    return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, n, value);
    return hipGetLastError();
}

hipError_t launch_write_tokens(int kv_f16, const WriteTokensArgs& a, hipStream_t stream) {
    if (a.n <= 0) return hipSuccess;
    dim3 grid(a.n, a.n_kv);
    if (kv_f16)
        hipLaunchKernelGGL(write_tokens_kernel<_Float16>, grid, dim3(128), 0, stream, a);
    else
        hipLaunchKernelGGL(write_tokens_kernel<float>, grid, dim3(128), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_rope_write(int kv_f16, const RopeWriteArgs& a, hipStream_t stream) {
    if (a.n <= 0) return hipSuccess;
    if (a.head_dim > 2 * kRopeMaxHalf || (a.head_dim & 1) || a.rope_dim < 2 || a.rope_dim > a.head_dim ||
        (a.rope_dim & 1))
        return hipErrorInvalidValue;
    const auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    const bool vec = a.head_dim % 8 == 0 && a.rope_dim % 8 == 0 && a.v_head_dim % 4 == 0 && al16(a.q) &&
                     al16(a.k) && al16(a.v) && al16(a.k_pool) && al16(a.v_pool);
    if (vec) {
        const int items = (a.n_heads + a.n_kv) * (a.head_dim / 8) + a.n_kv * (a.v_head_dim / 4);
        const dim3 grid(a.n, (items + 255) / 256);
        if (kv_f16)
            hipLaunchKernelGGL(rope_write_vec_kernel<_Float16>, grid, dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(rope_write_vec_kernel<float>, grid, dim3(256), 0, stream, a);
    } else if (kv_f16) {
        hipLaunchKernelGGL(rope_write_kernel<_Float16>, dim3(a.n), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(rope_write_kernel<float>, dim3(a.n), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_copy_block(int kv_f16, const CopyBlockArgs& a, hipStream_t stream) {
    dim3 grid(a.layers * a.n_kv);
    if (kv_f16)
        hipLaunchKernelGGL(copy_block_kernel<_Float16>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(copy_block_kernel<float>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gsp
