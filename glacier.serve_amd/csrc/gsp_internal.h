// Definitions shared by the host runtime and the gfx950 kernels of the
// paged-attention step.  Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gsp {

constexpr int kBlockSize = 16;    // tokens per KV page (PagedBlockPool.DefaultBlockSize)
constexpr int kDecodeWaves = 4;   // wave64s per decode workgroup
constexpr int kDecodeThreads = kDecodeWaves * 64;
constexpr int kMaxGroup = 8;      // query heads per KV head of the DPP decode kernel
constexpr int kMaxGroupMfma = 16; // query heads per KV head of the MFMA decode kernel (M/N tile)

// One split-KV work unit of the decode kernel: a contiguous range of logical
// pages of one query token.  The grid is (units, heads_kv); 32 bytes each.
struct DecodeUnit {
    int32_t qi;          // query token (row of q / out)
    int32_t bt_base;     // offset of the token's row table inside the packed ids
    int32_t page_begin;  // first logical page of the split
    int32_t page_end;    // one past the last logical page of the split
    int32_t ctx;         // tokens the query attends to: min(TokenCount, pos + 1)
    int32_t split;       // split index in [0, nsplit)
    int32_t nsplit;      // splits of this query token
    int32_t slot;        // first partial slot of this query token (nsplit > 1)
};
static_assert(sizeof(DecodeUnit) == 32, "DecodeUnit is packed as 8 int32");

struct DecodeArgs {
    const void* k_pool;
    const void* v_pool;
    int64_t block_stride;  // elements per block over all layers and heads
    int64_t layer_offset;  // layer * heads_kv * 16 * head_dim
    int64_t head_stride;   // 16 * head_dim
    const DecodeUnit* units;
    const int32_t* bt_ids;
    const float* q;        // [total_q][n_heads][head_dim]
    float* out;            // [total_q][n_heads][head_dim]
    float* part_o;         // [slot][n_heads][head_dim] unnormalised partial outputs
    float* part_ml;        // [slot][n_heads][2] running max (log2 units) and sum
    int32_t n_heads;
    int32_t n_kv;
    float scale_log2;      // attn_scale * log2(e)
};

// A query token whose pages were split over several units: its partials
// occupy slots [slot, slot + nsplit).  16 bytes each.
struct MergeItem {
    int32_t qi;
    int32_t slot;
    int32_t nsplit;
    int32_t pad;
};
static_assert(sizeof(MergeItem) == 16, "MergeItem is packed as 4 int32");

struct MergeArgs {
    const MergeItem* items;
    const float* part_o;
    const float* part_ml;
    float* out;
    int32_t n_heads;
    int32_t n_kv;
};

// Launches the DPP decode kernel instantiated for (head_dim, kv dtype, group <= 8).
hipError_t launch_decode(int head_dim, int kv_f16, int group, int num_units,
                         const DecodeArgs& a, hipStream_t stream);
// Launches the MFMA decode kernel for (head_dim, kv dtype); group <= 16.
hipError_t launch_decode_mfma(int head_dim, int kv_f16, int num_units, const DecodeArgs& a,
                              hipStream_t stream);
// Combines split partials into out, one workgroup per (item, KV head).
hipError_t launch_merge(int head_dim, int num_items, const MergeArgs& a, hipStream_t stream);

struct WriteTokensArgs {
    void* k_pool;
    void* v_pool;
    int64_t block_stride;
    int64_t layer_offset;
    int64_t head_stride;
    const int32_t* block_ids;  // [n]
    const int32_t* slots;      // [n]
    const float* k;            // [n][n_kv][d]
    const float* v;            // [n][n_kv][d]
    int32_t n;
    int32_t n_kv;
    int32_t head_dim;
};

hipError_t launch_write_tokens(int kv_f16, const WriteTokensArgs& a, hipStream_t stream);

struct CopyBlockArgs {
    void* k_pool;
    void* v_pool;
    int64_t block_stride;
    int64_t head_stride;
    int32_t src;
    int32_t dst;
    int32_t valid_tokens;  // already clamped to [1, 16]
    int32_t layers;
    int32_t n_kv;
    int32_t head_dim;
};

hipError_t launch_copy_block(int kv_f16, const CopyBlockArgs& a, hipStream_t stream);

}  // namespace gsp
