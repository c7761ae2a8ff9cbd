// Device page operations on the KV pool (gfx950): the batched Store scatter
// and the copy-on-write page copy.  Both are plain HBM-bound copies.
#include "gsp_internal.h"

namespace gsp {
namespace {

// PagedBlockPool.Store (PagedBlockPool.cs:151-161) for n tokens at once:
// token i, KV head h -> K/V[block_ids[i]][layer][h][slots[i]][:].  One
// workgroup per (token, head); fp32 -> fp16 rounds to nearest even.
template <typename KT>
__global__ __launch_bounds__(128) void write_tokens_kernel(WriteTokensArgs a) {
    const int i = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t dst = (int64_t)a.block_ids[i] * a.block_stride + a.layer_offset +
                        (int64_t)h * a.head_stride + (int64_t)a.slots[i] * a.head_dim;
    const int64_t src = ((int64_t)i * a.n_kv + h) * a.head_dim;
    KT* kd = static_cast<KT*>(a.k_pool) + dst;
    KT* vd = static_cast<KT*>(a.v_pool) + dst;
    for (int e = threadIdx.x; e < a.head_dim; e += blockDim.x) {
        kd[e] = static_cast<KT>(a.k[src + e]);
        vd[e] = static_cast<KT>(a.v[src + e]);
    }
}

// PagedBlockPool.CopyBlockData (PagedBlockPool.cs:304-327): the first
// valid_tokens slots of every (layer, KV head) page of `src` go to `dst`.
template <typename KT>
__global__ __launch_bounds__(256) void copy_block_kernel(CopyBlockArgs a) {
    const int lh = blockIdx.x;  // layer * n_kv + head: pages are consecutive
    const int64_t n = (int64_t)a.valid_tokens * a.head_dim;
    const int64_t off = (int64_t)lh * a.head_stride;
    const KT* ks = static_cast<const KT*>(a.k_pool) + (int64_t)a.src * a.block_stride + off;
    const KT* vs = static_cast<const KT*>(a.v_pool) + (int64_t)a.src * a.block_stride + off;
    KT* kd = static_cast<KT*>(a.k_pool) + (int64_t)a.dst * a.block_stride + off;
    KT* vd = static_cast<KT*>(a.v_pool) + (int64_t)a.dst * a.block_stride + off;
    for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
        kd[e] = ks[e];
        vd[e] = vs[e];
    }
}

}  // namespace

hipError_t launch_write_tokens(int kv_f16, const WriteTokensArgs& a, hipStream_t stream) {
    if (a.n <= 0) return hipSuccess;
    dim3 grid(a.n, a.n_kv);
    if (kv_f16)
        hipLaunchKernelGGL(write_tokens_kernel<_Float16>, grid, dim3(128), 0, stream, a);
    else
        hipLaunchKernelGGL(write_tokens_kernel<float>, grid, dim3(128), 0, stream, a);
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
