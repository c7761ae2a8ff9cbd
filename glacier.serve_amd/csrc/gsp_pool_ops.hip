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
// with block id -1 has no slot and is skipped.
template <typename KT>
__global__ __launch_bounds__(128) void write_tokens_kernel(WriteTokensArgs a) {
    const int i = blockIdx.x;
    const int h = blockIdx.y;
    if (a.block_ids[i] < 0) return;
    const int64_t blk = a.block_ids[i];
    const int64_t slot = a.slots[i];
    KT* kd = static_cast<KT*>(a.k_pool) + blk * a.block_stride + a.layer_offset + h * a.head_stride + slot * a.head_dim;
    KT* vd = static_cast<KT*>(a.v_pool) + blk * a.v_block_stride + a.v_layer_offset + h * a.v_head_stride +
             slot * a.v_head_dim;
    const float* ks = a.k + ((int64_t)i * a.n_kv + h) * a.head_dim;
    const float* vs = a.v + ((int64_t)i * a.n_kv + h) * a.v_head_dim;
    for (int e = threadIdx.x; e < a.head_dim; e += blockDim.x) kd[e] = static_cast<KT>(ks[e]);
    for (int e = threadIdx.x; e < a.v_head_dim; e += blockDim.x) vd[e] = static_cast<KT>(vs[e]);
}

// QuantKernels.RoPE then PagedBlockPool.Store for n tokens
// (PagedTransformerRunner.cs:253-267, 437-452, 620-634), one workgroup per
// token.  Pair j of every head turns by pos * base^(-2j/d) (Su et al.,
// RoFormer): the angle is formed and reduced to [-pi, pi] in fp64, so it
// stays exact at long positions, and its cosine and sine are taken once per
// token in fp32.  Q heads are rotated in place, K heads are rotated into the
// pool slot and V is stored as is; fp16 pools round to nearest even.  A token
// with block id -1 has no slot: its Q is rotated, its K and V are not stored.
template <typename KT>
__global__ __launch_bounds__(256) void rope_write_kernel(RopeWriteArgs a) {
    __shared__ float cs[kRopeMaxHalf][2];
    const int i = blockIdx.x;
    const int d = a.head_dim;
    const int half = d >> 1;
    const double pos = (double)a.positions[i];
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
        const double ang = pos * exp2(-(2.0 * j / d) * a.log2_base);
        const double r = ang - 6.283185307179586 * rint(ang * 0.15915494309189535);
        float s, c;
        sincosf((float)r, &s, &c);
        cs[j][0] = c;
        cs[j][1] = s;
    }
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
    for (int idx = threadIdx.x; stored && idx < a.n_kv * dv; idx += blockDim.x) {
        const int hk = idx / dv;
        const int e = idx - hk * dv;
        static_cast<KT*>(a.v_pool)[vdst + (int64_t)hk * a.v_head_stride + e] =
            static_cast<KT>(a.v[((int64_t)i * a.n_kv + hk) * dv + e]);
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

}  // namespace

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
    if (a.head_dim > 2 * kRopeMaxHalf || (a.head_dim & 1)) return hipErrorInvalidValue;
    if (kv_f16)
        hipLaunchKernelGGL(rope_write_kernel<_Float16>, dim3(a.n), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(rope_write_kernel<float>, dim3(a.n), dim3(256), 0, stream, a);
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
