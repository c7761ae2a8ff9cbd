// Definitions shared by the host runtime and the gfx950 kernels of the
// paged-attention step.  Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "gsp_step_format.h"

namespace gsp {

struct DecodeArgs {
    const void* k_pool;
    const void* v_pool;
    int64_t block_stride;  // K elements per block over all layers and heads
    int64_t layer_offset;  // layer * heads_kv * block_size * head_dim
    int64_t head_stride;   // block_size * head_dim
    int64_t v_block_stride;  // the same for V (v_head_dim per slot)
    int64_t v_layer_offset;
    int64_t v_head_stride;
    // Workgroup b runs unit b first, then units [bin_rest[b], bin_rest[b + 1]):
    // the first unit of every bin sits at the bin's own index, so a workgroup
    // can fetch it without waiting for the offsets.
    const DecodeUnit* units;
    const int32_t* bin_rest;     // [num_bins + 1], bin_rest[0] == num_bins
    const int32_t* bt_ids;
    const float* q;        // [total_q][n_heads][head_dim]
    float* out;            // [total_q][n_heads][head_dim]
    // Split-KV workspace, per tile of heads (grid.y; one tile for groups up
    // to 16): partials [tile][slot][slot_heads][v_head_dim] and
    // [tile][slot][slot_heads][2] (running max in log2 units, sum), counters
    // [tile][total_q][n_kv] of splits finished, zero between launches.
    float* part_o;
    float* part_ml;
    int32_t* counters;
    int32_t n_heads;
    int32_t n_kv;
    int32_t group;         // query heads per KV head
    float scale_log2;      // attn_scale * log2(e)
    int32_t head_dim;      // K/Q width
    int32_t v_head_dim;    // V/out width
    int32_t block_size;    // tokens per page, 1..16
    int32_t tile_pages;    // pages per decode tile: 16 / block_size for 4- and 8-token pages, else 1
    int32_t total_q;
    int32_t num_slots;     // partial slots per tile
    int32_t slot_heads;    // heads per partial slot: min(group, 16)
};

struct PrefillArgs {
    const void* k_pool;
    const void* v_pool;
    int64_t block_stride;
    int64_t layer_offset;
    int64_t head_stride;
    const PrefillTile* tiles;
    const int32_t* bt_ids;
    const float* q;        // [total_q][n_heads][head_dim]
    float* out;            // [total_q][n_heads][head_dim]
    int32_t n_heads;
    int32_t n_kv;
    int32_t group;         // query heads per KV head (any; grid.y covers them 8, or for groups up to 4, 4 at a time)
    float scale_log2;
    // fp32 pages only: the step's split records (launch_prefill_split, this
    // layer), PrefillTile.rec0 being the first record of the tile's row and KV
    // head; null: each tile splits the pages it reads itself.
    const unsigned char* records;
};

struct PrefillSplitArgs {
    const void* k_pool;
    const void* v_pool;
    int64_t block_stride;
    int64_t layer_offset;
    int64_t head_stride;
    const PrefillSplitItem* items;
    const int32_t* bt_ids;
    unsigned char* records;
};

// Bytes of one split record (one page pair, one KV head) for head_dim 64 or 128 (else 0).
int prefill_record_bytes(int head_dim);
// Writes the split records of fp32 pages: grid (max_pairs, num_items).
hipError_t launch_prefill_split(int head_dim, int num_items, int max_pairs, const PrefillSplitArgs& a,
                                hipStream_t stream);

// Launches the MFMA prefill kernel for (head_dim, kv dtype); with a.records
// (fp32 pages) the tiles read the split records.
hipError_t launch_prefill_mfma(int head_dim, int kv_f16, int num_tiles, const PrefillArgs& a, hipStream_t stream);

// Launches a step with both decode bins and prefill tiles as one kernel (the
// matrix-core decode of the fixed shapes, head_dim == v_head_dim in {64, 128},
// 16-token pages, and the prefill tiles).  DecodeArgs and PrefillArgs are
// those of the two separate launches.
hipError_t launch_mixed_mfma(int head_dim, int kv_f16, int num_bins, int num_tiles, const DecodeArgs& da,
                             const PrefillArgs& pa, hipStream_t stream);

// Launches the DPP decode kernel instantiated for (head_dim, kv dtype, group <= 8),
// one workgroup per bin.
hipError_t launch_decode(int head_dim, int kv_f16, int num_bins, const DecodeArgs& a, hipStream_t stream);
// Launches the MFMA decode kernel, one workgroup per (bin, tile of 16 heads).
// head_dim == v_head_dim in {64, 128} with 16-token pages take the fixed-shape
// instantiations; any other even head_dim / v_head_dim <= 256 and block size
// <= 16 take the general ones.
hipError_t launch_decode_mfma(int kv_f16, int num_bins, const DecodeArgs& a, hipStream_t stream);

struct WriteTokensArgs {
    void* k_pool;
    void* v_pool;
    int64_t block_stride;
    int64_t layer_offset;
    int64_t head_stride;
    int64_t v_block_stride;
    int64_t v_layer_offset;
    int64_t v_head_stride;
    const int32_t* block_ids;  // [n]; -1: no slot, nothing stored
    const int32_t* slots;      // [n]
    const float* k;            // [n][n_kv][head_dim]
    const float* v;            // [n][n_kv][v_head_dim]
    int32_t n;
    int32_t n_kv;
    int32_t head_dim;
    int32_t v_head_dim;
};

hipError_t launch_write_tokens(int kv_f16, const WriteTokensArgs& a, hipStream_t stream);

constexpr int kRopeMaxHalf = 128;  // head_dim <= 256

struct RopeWriteArgs {
    void* k_pool;
    void* v_pool;
    int64_t block_stride;
    int64_t layer_offset;
    int64_t head_stride;
    int64_t v_block_stride;
    int64_t v_layer_offset;
    int64_t v_head_stride;
    const int32_t* positions;  // [n]
    const int32_t* block_ids;  // [n]
    const int32_t* slots;      // [n]
    float* q;                  // [n][n_heads][d], rotated in place (n_heads 0: none)
    const float* k;            // [n][n_kv][d], rotated into the pool
    const float* v;            // [n][n_kv][v_head_dim], stored as is
    const double* freq;        // [rope_dim / 2] angle per position of each pair, or NULL:
    double log2_base;          // then pair j turns by freq_base^(-2j / rope_dim), log2(freq_base) here
    int32_t n;
    int32_t n_heads;
    int32_t n_kv;
    int32_t head_dim;
    int32_t v_head_dim;
    int32_t style;             // GSP_ROPE_PAIRS or GSP_ROPE_HALVES
    int32_t rope_dim;          // dims rotated (even, <= head_dim); the rest pass through
    float mscale;              // scale of the rotated dims
};

hipError_t launch_rope_write(int kv_f16, const RopeWriteArgs& a, hipStream_t stream);

// Projection GEMM (gsp_matmul.hip): y[b][o] = sum_i W[o][i] x[b][i].
constexpr int kWeightF32 = 0;   // GGUF type ids
constexpr int kWeightQ8_0 = 8;
constexpr int kWeightQ4_K = 12;  // super-blocks of 256 weights, 144 bytes
constexpr int kWeightQ6_K = 14;  // super-blocks of 256 weights, 210 bytes
struct MatmulArgs {
    const void* w;       // out_dim rows of in_dim weights (F32, or Q8_0 blocks of 34 bytes)
    const float* x;      // [batch][in_dim]
    float* y;            // [batch][out_dim]
    float* split_out;    // [splits][batch][out_dim] partials when splits > 1, else null
    int32_t w_type;
    int32_t in_dim;      // a multiple of 64
    int32_t out_dim;
    int32_t batch;
    int32_t splits;            // K ranges over grid.z
    int32_t chunks_per_split;  // 64-wide K chunks per range
    // Q8_0 path: x as scaled fp16 pairs, [batch][in_dim] each, and each row's exponent.
    void* xh;
    void* xl;
    int32_t* xexp;
    // Small-batch form (batch <= 64): one counter per 64 weight rows, zero between launches.
    int32_t* counters;
    // Small-batch Q4_K: the pre-pass's block sums of the scaled x, splits x 2 chunks_per_split x 64 floats.
    float* xsum;
};
hipError_t launch_matmul(const MatmulArgs& a, hipStream_t stream);
// The small-batch form (batch <= 64, Q8_0, Q4_K or Q6_K weights): the x pre-pass in
// tile order (xh: matmul_small_x_halves halves, xexp: splits x batch
// exponents, one per K range of each row; for Q4_K also xsum), then one
// product kernel that merges its K ranges itself (Q6_K: chunks_per_split
// even, so that ranges start on a super-block half).  A workgroup stages
// matmul_small_chunks(batch) chunks of its range at a time (longer ranges take
// several passes).  Needs chunks_per_split <= matmul_small_range_chunks_max(),
// splits <= matmul_small_max_splits(batch) and, with splits > 1, split_out
// holding splits x batch x (64 * tiles) floats (16-byte aligned) and one
// zeroed counter per tile of 64 weight rows.
hipError_t launch_matmul_small(const MatmulArgs& a, hipStream_t stream);
int matmul_small_chunks(int batch);
int matmul_small_range_chunks_max();
int matmul_small_max_splits(int batch);
int64_t matmul_small_x_halves(int batch, int in_dim);

struct CopyBlockArgs {
    void* k_pool;
    void* v_pool;
    int64_t block_stride;
    int64_t head_stride;
    int64_t v_block_stride;
    int64_t v_head_stride;
    int32_t src;
    int32_t dst;
    int32_t valid_tokens;  // already clamped to [1, block_size]
    int32_t layers;
    int32_t n_kv;
    int32_t head_dim;
    int32_t v_head_dim;
};

hipError_t launch_copy_block(int kv_f16, const CopyBlockArgs& a, hipStream_t stream);

// Sets n int32 words at p to `value` with a kernel (capturable, unlike hipMemsetAsync).
hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t stream);

// Copies n16 16-byte words from src (device-visible pinned host memory, both
// 16-byte aligned) to dst with a kernel on `stream`.
hipError_t launch_upload_step(const void* src, void* dst, int64_t n16, hipStream_t stream);

// Fixed device scratch of the allocation-free attention entry point
// (gsp_noalloc.hip): one array per GPU, its address looked up once per device.
hipError_t noalloc_setup(int device);
// The device address of `device`'s scratch array, or null before noalloc_setup.
void* noalloc_scratch(int device);

}  // namespace gsp
