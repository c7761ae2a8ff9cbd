// Matrix-core (MFMA) decode kernel of the paged-attention step, gfx950.  The
// device code and its description are in gsp_decode_body.h.
#include "gsp_decode_body.h"

namespace gsp {
namespace {

template <int D, typename KT, int MODE>
__global__ __launch_bounds__(kDecodeThreads, D >= 256 ? 1 : 2) void paged_decode_mfma_kernel(DecodeArgs a) {
    __shared__ EpilogueLds<D, kMaxGroupMfma> sh;
    decode_bins_body<D, KT, MODE>(a, sh, blockIdx.x, blockIdx.y);
}

template <int D, typename KT, int MODE>
void launch_one(dim3 grid, const DecodeArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL((paged_decode_mfma_kernel<D, KT, MODE>), grid, dim3(kDecodeThreads), 0, stream, a);
}

template <typename KT>
hipError_t launch_typed(dim3 grid, const DecodeArgs& a, hipStream_t stream) {
    const int d = a.head_dim, dv = a.v_head_dim;
    // A tile of several pages only for 4- and 8-token pages (16 rows).
    if (a.tile_pages < 1 || (a.tile_pages > 1 && ((a.block_size != 4 && a.block_size != 8) ||
                                                  a.block_size * a.tile_pages != kTileTokens)))
        return hipErrorInvalidValue;
    if (d == dv && a.block_size == kBlockSize && (d == 64 || d == 128)) {
        if (d == 128)
            launch_one<128, KT, kExact>(grid, a, stream);
        else
            launch_one<64, KT, kExact>(grid, a, stream);
    } else if (d < 1 || dv < 1 || d > 256 || dv > 256 || a.block_size < 1 || a.block_size > kTileTokens) {
        return hipErrorInvalidValue;
    } else if (d % 2 || dv % 2) {
        launch_one<256, KT, kVec1>(grid, a, stream);
    } else if (d % 4 == 0 && dv % 4 == 0) {
        const int w = max(d, dv);
        if (w <= 64)
            launch_one<64, KT, kVec4>(grid, a, stream);
        else if (w <= 128)
            launch_one<128, KT, kVec4>(grid, a, stream);
        else
            launch_one<256, KT, kVec4>(grid, a, stream);
    } else {
        launch_one<256, KT, kVec2>(grid, a, stream);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_mfma(int kv_f16, int num_bins, const DecodeArgs& a, hipStream_t stream) {
    if (num_bins <= 0) return hipSuccess;
    if (a.group < 1) return hipErrorInvalidValue;
    const dim3 grid(num_bins, (a.group + kDecodeTileHeads - 1) / kDecodeTileHeads);
    return kv_f16 ? launch_typed<_Float16>(grid, a, stream) : launch_typed<float>(grid, a, stream);
}

}  // namespace gsp
