// The packed step's format: the constants and the records that the host
// packer (gsp_step_plan.cpp) writes and the gfx950 kernels read.  No HIP
// here, so the packer also builds with a plain host compiler (the sanitizer
// builds under tests/native).
#pragma once

#include <cstdint>

namespace gsp {

constexpr int kBlockSize = 16;    // tokens per KV page (PagedBlockPool.DefaultBlockSize)
constexpr int kDecodeWaves = 4;   // wave64s per decode workgroup
constexpr int kDecodeThreads = kDecodeWaves * 64;
constexpr int kMaxGroup = 8;      // query heads per KV head of the DPP decode kernel
constexpr int kMaxGroupMfma = 16; // query heads per KV head of the MFMA decode kernel (M/N tile)
constexpr int kMaxSplits = 256;   // split-KV units per (query token, KV head) pair

// One unit of decode work, one workgroup each: a contiguous range of logical
// pages of one (query token, KV head) pair.  Units are ordered longest first
// so the hardware's in-order dispatch schedules them like LPT.  64 bytes each.
struct DecodeUnit {
    int32_t qi;          // query token (row of q / out)
    int32_t bt_base;     // offset of the token's row table inside the packed ids
    int32_t page_begin;  // first logical page of the unit
    int32_t page_end;    // one past the last logical page of the unit
    int32_t ctx;         // tokens the query attends to: min(TokenCount, pos + 1)
    int32_t kvh;         // KV head
    int32_t slot;        // first partial slot of the pair (-1 when nsplit == 1)
    int32_t split_info;  // split index | nsplit << 16
    int32_t first_blk[kDecodeWaves];   // block of each wave's first page (-1: none) and of
    int32_t second_blk[kDecodeWaves];  // its second, so a unit's first two page loads per
                                       // wave need no table lookup
};
static_assert(sizeof(DecodeUnit) == 64, "DecodeUnit is packed as 16 int32");

// Query heads per decode tile (the matrix-core kernel's 16-wide N): larger
// GQA groups run as several tiles over grid.y.
constexpr int kDecodeTileHeads = 16;

// One prefill tile, one workgroup per (tile, group of up to 8 query heads):
// up to 16 consecutive query tokens of one row against one KV head.  Query
// token j of the tile attends to min(token_count, pos0 + j + 1) tokens.
struct PrefillTile {
    int32_t qi0;          // first query token of the tile (row of q / out)
    int32_t bt_base;      // offset of the row's table inside the packed ids
    int32_t pos0;         // position of the first query token
    int32_t ntok;         // query tokens in the tile, 1..16
    int32_t token_count;  // the row's BlockTable.TokenCount
    int32_t pages;        // ceil(min(token_count, pos0 + ntok) / 16): pages the tile reads
    int32_t kvh;          // KV head
    int32_t rec0;         // first split record of the tile's row and KV head (fp32 pages)
};
static_assert(sizeof(PrefillTile) == 32, "PrefillTile is packed as 8 int32");

constexpr int kPrefillTileTokens = 16;  // query tokens per tile (MFMA N dimension)
constexpr int kPrefillHeads = 8;        // query heads per prefill workgroup (two per wave)

// One (row, KV head) of the split records: records rec0 .. rec0 + pairs - 1
// hold its page pairs, pairs = ceil(ceil(ctx_last / 16) / 2).
struct PrefillSplitItem {
    int32_t bt_base;   // offset of the row's table inside the packed ids
    int32_t ctx_last;  // tokens of the row its tiles read: min(TokenCount, pos + q_len)
    int32_t kvh;
    int32_t rec0;
};
static_assert(sizeof(PrefillSplitItem) == 16, "PrefillSplitItem is packed as 4 int32");

// Packed step header, in int32 words from the start of the step image.
enum : int {
    kHdrRows = 0,
    kHdrTotalQ,
    kHdrPages,
    kHdrUnits,
    kHdrTarget,
    kHdrSlots,
    kHdrMaxId,
    kHdrPairsSplit,
    kHdrHeadsKv,
    kHdrTiles,
    kHdrBins,
    kHdrWords = 16
};

}  // namespace gsp
