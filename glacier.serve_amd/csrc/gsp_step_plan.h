// Host packer of the paged-attention step, without HIP: validation of an
// engine step against the reference's bounds and the pool, the split-KV unit
// plan, the prefill tiles, the decode bins and the step image the kernels
// read.  gsp_step_pack (gsp_runtime.cpp) runs it and uploads the image; the
// sanitizer builds under tests/native drive it directly.
#pragma once

#include <cstddef>
#include <cstdint>
#include <utility>
#include <vector>

#include "../../include/glacier_paged.h"
#include "gsp_step_format.h"

namespace gsp {

// The pool geometry a step is planned for.
struct PlanPool {
    int32_t total_blocks = 0;
    int32_t layers = 1;
    int32_t heads_kv = 0;
    int32_t head_dim = 0;
    int32_t v_head_dim = 0;
    int32_t block_size = 0;
    int32_t kv_dtype = GSP_KV_F32;
};

// The context's tuning choices (gsp_set_*) and the device's CU count.
struct PlanOptions {
    int32_t num_cus = 1;
    int32_t split_pages_override = 0;
    int32_t decode_bins_override = 0;
    int32_t prefill_path = GSP_PREFILL_AUTO;
    int32_t prefill_split = GSP_SPLIT_RECORDS;
};

// A planned step: its image (int32 words, uploaded as is) and the sizes the
// launches need.  The image holds, at the word offsets below: the header
// (kHdr*), row_offsets [B + 1], the packed ids, ctx_lens [total_q], the write
// slots [3 * total_q] (position, block or -1, slot), the decode units (64
// bytes each, unit b first of bin b), the prefill tiles, the split-record
// items and bin_rest [num_bins + 1].
struct StepPlan {
    std::vector<int32_t> image;
    size_t off_rows = 0, off_ids = 0, off_ctx = 0, off_wr = 0, off_units = 0, off_tiles = 0, off_split = 0,
           off_bins = 0;
    int32_t num_rows = 0;
    int64_t total_q = 0;
    int64_t packed_pages = 0;
    int64_t kv_tokens = 0;
    int32_t num_units = 0;
    int32_t num_bins = 0;
    int32_t num_tiles = 0;
    int64_t num_slots = 0;
    int64_t pairs_split = 0;
    int32_t target = 0;            // largest unit, in pages
    int32_t num_split_items = 0;   // (row, KV head) items of the split records
    int32_t split_max_pairs = 0;
    int64_t num_records = 0;       // split records (fp32 prefill tiles)
    int64_t tiled_queries = 0;
    int64_t tiled_pairs = 0;
    int32_t max_id = -1;           // largest pool block id the step reads
    bool tileable = false;         // the pool's shape takes prefill tiles
    // Kernel pages: the packed ids and the units count pages of page_tokens
    // (<= 16) tokens.  pool_page_split == 1: they are the pool's pages and
    // blocks.  Above 1, each pool page is that many kernel pages, with ids
    // block * (layers * heads_kv * pool_page_split) + sub-page, so the kernels
    // take a page stride of page_tokens * head_dim (v_head_dim for V).
    int32_t page_tokens = 0;
    int32_t pool_page_split = 1;
    // Decode units count tiles of tile_pages kernel pages (2 for 8-token and
    // 4 for 4-token pages, else 1): their page_begin / page_end and
    // first_blk / second_blk (the tile's first page) are in tiles.
    int32_t tile_pages = 1;
};

class StepPlanner {
public:
    // Validates `desc` for `pool` (the reference's throws,
    // PagedAttentionKernel.cs:34-39, plus the table and pool bounds) and plans
    // it into `out`.  GSP_OK, or GSP_E_INVALID_ARG with the message set and
    // `out` unspecified (GSP_E_UNSUPPORTED for pool pages above 16 tokens whose
    // kernel page ids would not fit 32 bits).
    int plan(const PlanPool& pool, const gsp_step_desc* desc, const PlanOptions& opt, StepPlan& out);

private:
    int32_t assign_bins(int64_t bins_max, bool pair);

    // Split size chosen for the last step shape (reused while the work drifts < 3%).
    int32_t cached_target_ = 0;
    int64_t cached_tasks_ = 0;
    int32_t cached_heads_kv_ = 0;
    int64_t cached_queries_ = 0;
    int64_t cached_bins_ = 0;

    // Scratch reused across steps.
    std::vector<DecodeUnit> units_;    // in the order they were built
    std::vector<int32_t> unit_order_;  // unit indices, longest first (stable)
    std::vector<int32_t> unit_place_;  // unit indices in their packed order (assign_bins)
    std::vector<int32_t> len_count_;   // counting sort of unit_order_
    std::vector<int32_t> bin_units_;   // [num_bins + 1] offsets of each bin's units after its first
    std::vector<int32_t> unit_bin_;
    std::vector<std::pair<int64_t, int32_t>> bin_heap_;
    std::vector<int32_t> bin_cursor_;
    std::vector<int64_t> bin_load_;
    std::vector<PrefillTile> tiles_;
    std::vector<PrefillSplitItem> split_items_;
    std::vector<int32_t> q_ctx_;
    std::vector<int32_t> query_pages_;
    std::vector<int32_t> voffs_, vids_;  // row tables in kernel pages (pool pages above 16 tokens)
    std::vector<int64_t> sim_count_, sim_heap_;
};

}  // namespace gsp
