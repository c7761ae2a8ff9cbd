// Host packer of the paged-attention step (see gsp_step_plan.h).  Plain C++,
// no HIP: gsp_step_pack runs it and uploads the image; tests/native builds it
// under AddressSanitizer and UndefinedBehaviorSanitizer.
#include "gsp_step_plan.h"

#include <algorithm>
#include <climits>
#include <cstring>
#include <functional>

#include "gsp_status.h"

namespace gsp {
namespace {

// Decode schedule.  The decode kernel is persistent: one workgroup per bin,
// and each bin's units run back to back while the next unit's first pages
// are already in flight.  The host packs units into bins longest first (LPT
// list scheduling).  Within a bin, split pieces go first and whole pairs
// last, so split merges finish while other work still streams rather than in
// the kernel's tail.  Two bins per CU (the decode kernels' occupancy) keep a
// second workgroup streaming while the first one is in a unit epilogue; one
// workgroup alone can draw the CU's full share of HBM bandwidth, so the split
// size is scored per CU.  A unit costs its pages plus a fixed transition; a
// split piece also pays for publishing its partial and for its share of the
// merge.
constexpr int kDecodeBinsPerCu = 2;
constexpr int64_t kUnitCostPages = 1;
constexpr int64_t kSplitCostPages = 3;
constexpr int32_t kSplitCandidates[] = {8,   12,  16,  20,  24,  32,  40,  48,  64,  80,   96,
                                        128, 160, 192, 256, 384, 512, 768, 1024, 1536, 2048};

// A step with few pages per workgroup is latency-bound: a unit of at most
// four pages per wave streams in about two round trips, and a split would add
// its publish, count and merge round trips for nothing (config 1 measured
// 6.8 us whole against 7.6 us split).
constexpr int64_t kWholePairMaxPages = 4 * gsp::kDecodeWaves;
constexpr int64_t kUnderloadPagesPerBin = 4;

int64_t unit_cost(int64_t pages, bool split) { return pages + kUnitCostPages + (split ? kSplitCostPages : 0); }

// Makespan (in pages) of LPT-packing the units that `target` produces from
// the per-query page counts into `bins` bins.
int64_t simulate_split(const std::vector<int32_t>& pages, int32_t heads_kv, int32_t target, int64_t bins,
                       std::vector<int64_t>& count, std::vector<int64_t>& heap) {
    // count[2s] whole pairs of s pages, count[2s + 1] split pieces of s pages.
    count.assign(2 * ((size_t)target + 1), 0);
    int32_t longest = 0;
    for (int32_t P : pages) {
        const int32_t ns = std::min((P + target - 1) / target, gsp::kMaxSplits);
        const int32_t base = P / ns, extra = P % ns;
        const int sp = ns > 1 ? 1 : 0;
        // Pieces of base + 1 pages exist only when extra > 0, and then base < target.
        if (extra) count[2 * ((size_t)base + 1) + sp] += (int64_t)extra * heads_kv;
        count[2 * (size_t)base + sp] += (int64_t)(ns - extra) * heads_kv;
        longest = std::max(longest, base + (extra ? 1 : 0));
    }
    heap.clear();
    for (int32_t s = longest; s >= 1; --s) {
        for (int sp = 1; sp >= 0; --sp) {
            const int64_t cost = unit_cost(s, sp == 1);
            for (int64_t c = count[2 * (size_t)s + sp]; c > 0; --c) {
                if ((int64_t)heap.size() < bins) {
                    heap.push_back(-cost);  // min-heap through negated loads
                    std::push_heap(heap.begin(), heap.end());
                } else {
                    std::pop_heap(heap.begin(), heap.end());
                    heap.back() -= cost;
                    std::push_heap(heap.begin(), heap.end());
                }
            }
        }
    }
    int64_t worst = 0;
    for (int64_t x : heap) worst = std::max(worst, -x);
    return worst;
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Rows of at least this many query tokens run as prefill tiles by default:
// a tile reads each K/V page once for 16 query tokens, while shorter rows keep
// the decode kernel's split-KV parallelism over long prefixes.
constexpr int32_t kPrefillAutoMinQ = 16;

bool row_is_tiled(int32_t path, int32_t q_len, bool tileable) {
    if (!tileable || path == GSP_PREFILL_PER_TOKEN || q_len < 2) return false;
    return path == GSP_PREFILL_TILES || q_len >= kPrefillAutoMinQ;
}

}  // namespace


// Packs the longest-first units into bins, one decode workgroup each.
//  - LPT: each unit goes to the least-loaded bin (ties to the lowest).  With
//    `pair` (a grid of two workgroups per CU) the LPT runs over `nb / 2` CU
//    bins and each CU bin's units are then dealt to its workgroups c and
//    c + nb / 2, each unit to the lighter of the two.  In-order dispatch puts
//    those two workgroups on one CU, where they share its bandwidth, so what
//    must balance is their sum; should they land apart, each still holds
//    about half of a balanced CU bin.  Pairing needs two units per CU bin.
//  - Within a bin, split pieces run first and whole pairs last, each group
//    keeping the longest-first order, so merges finish before the tail.
// Works on unit indices: unit_order (longest first) in, unit_place out.
// Layout: unit_place[b] is bin b's first unit; the other units follow, bin by
// bin, with bin b's at [bin_units[b], bin_units[b + 1]).  No bin is empty.
// Returns the bin count.
int32_t StepPlanner::assign_bins(int64_t bins_max, bool pair) {
    const std::vector<int32_t>& ord = unit_order_;
    const size_t n = ord.size();
    const int32_t nb = (int32_t)std::min<int64_t>(bins_max, (int64_t)n);
    bin_units_.assign((size_t)nb + 1, 0);
    if (nb == 0) return 0;
    pair = pair && nb == bins_max && nb % 2 == 0;
    const int32_t nl = pair ? nb / 2 : nb;  // bins of the LPT
    auto& heap = bin_heap_;
    heap.clear();
    for (int32_t b = 0; b < nl; ++b) heap.emplace_back(0, b);
    const std::greater<std::pair<int64_t, int32_t>> later;
    std::make_heap(heap.begin(), heap.end(), later);
    unit_bin_.resize(n);
    auto& count = bin_cursor_;
    count.assign((size_t)nl, 0);
    for (size_t i = 0; i < n; ++i) {
        const DecodeUnit& u = units_[(size_t)ord[i]];
        std::pop_heap(heap.begin(), heap.end(), later);
        const int32_t b = heap.back().second;
        unit_bin_[i] = b;
        count[(size_t)b] += 1;
        heap.back().first += unit_cost(u.page_end - u.page_begin, (u.split_info >> 16) > 1);
        std::push_heap(heap.begin(), heap.end(), later);
    }
    if (pair) {
        for (int32_t b = 0; b < nl; ++b)
            if (count[(size_t)b] < 2) return assign_bins(bins_max, false);
        auto& load = bin_load_;
        load.assign((size_t)nb, 0);
        for (int pass = 0; pass < 2; ++pass)
            for (size_t i = 0; i < n; ++i) {
                const DecodeUnit& u = units_[(size_t)ord[i]];
                const bool split = (u.split_info >> 16) > 1;
                if (split != (pass == 0)) continue;
                const int32_t c = unit_bin_[i];
                const int32_t w = load[(size_t)c] <= load[(size_t)(c + nl)] ? c : c + nl;
                unit_bin_[i] = w;
                load[(size_t)w] += unit_cost(u.page_end - u.page_begin, split);
            }
        for (size_t i = 0; i < n; ++i) bin_units_[(size_t)unit_bin_[i] + 1] += 1;
    } else {
        for (int32_t b = 0; b < nb; ++b) bin_units_[(size_t)b + 1] = count[(size_t)b];
    }
    // bin_units[b + 1] holds bin b's unit count: its first unit goes to slot b,
    // the rest to the bin's run after the nb first units.
    bin_units_[0] = nb;
    for (int32_t b = 0; b < nb; ++b) bin_units_[(size_t)b + 1] += bin_units_[(size_t)b] - 1;
    auto& cursor = bin_cursor_;
    cursor.assign((size_t)nb, -1);  // -1: the bin's first unit is still to place
    unit_place_.resize(n);
    for (int pass = 0; pass < 2; ++pass) {
        const bool want_split = pass == 0;
        for (size_t i = 0; i < n; ++i) {
            const DecodeUnit& u = units_[(size_t)ord[i]];
            if (((u.split_info >> 16) > 1) != want_split) continue;
            const int32_t b = unit_bin_[i];
            int32_t& cur = cursor[(size_t)b];
            if (cur < 0) {
                unit_place_[(size_t)b] = ord[i];
                cur = bin_units_[(size_t)b];
            } else {
                unit_place_[(size_t)cur++] = ord[i];
            }
        }
    }
    return nb;
}

int StepPlanner::plan(const PlanPool& pool, const gsp_step_desc* desc, const PlanOptions& opt, StepPlan& out) {
    if (!desc) return fail(GSP_E_INVALID_ARG, "desc is NULL");
    const PlanPool& pd = pool;
    const int32_t B = desc->num_rows;
    if (B < 0) return fail(GSP_E_INVALID_ARG, "num_rows must be >= 0 (got %d)", B);
    if (desc->max_seq_len <= 0)
        return fail(GSP_E_INVALID_ARG, "maxSeqLen must be positive (got %d)", desc->max_seq_len);
    if (B > 0 && (!desc->positions || !desc->token_counts || !desc->bt_offsets || !desc->bt_ids))
        return fail(GSP_E_INVALID_ARG, "positions/token_counts/bt_offsets/bt_ids must not be NULL");
    const int32_t L = desc->max_seq_len;
    const int32_t H = pd.heads_kv;
    if (pd.block_size < 1) return fail(GSP_E_INVALID_ARG, "blockSize must be >= 1 (got %d)", pd.block_size);
    // The kernels read pages of at most 16 tokens.  A pool page of pbs > 16
    // tokens is read as r = pbs / bs kernel pages of bs tokens (bs the largest
    // divisor of pbs up to 16): kernel page k of a row is sub-page k % r of
    // pool page k / r, and its id b * (layers * heads_kv * r) + k % r times a
    // kernel page stride of bs * head_dim addresses exactly that sub-page in
    // the reference layout [block][layer][head][slot][dim]
    // (PagedBlockPool.cs:77-83).  Validation below is in pool pages.
    const int32_t pbs = pd.block_size;
    int32_t bs = std::min(pbs, kBlockSize);
    while (pbs % bs) --bs;
    const int32_t r = pbs / bs;
    // Decode units count 16-token tiles: a tile of 4- or 8-token pages is the
    // tile_pages = 16 / bs consecutive pages of the row (the general kernels
    // read each from its own block), so a wave's tile carries no empty rows.
    // Other page sizes take one page per tile.
    const int32_t m = (r == 1 && (bs == 4 || bs == 8)) ? kBlockSize / bs : 1;
    const int32_t tt = bs * m;  // tokens per decode tile
    const int64_t vfactor = (int64_t)std::max(1, pd.layers) * H * r;
    if (r > 1 && ((int64_t)pd.total_blocks - 1) * vfactor + (r - 1) > INT32_MAX)
        return fail(GSP_E_UNSUPPORTED, "%d blocks of %d-token pages: too many kernel pages for 32-bit ids",
                    pd.total_blocks, pbs);
    // Prefill tiles serve 16-token pages of equal K and V widths 64 or 128;
    // rows of other pools run as per-query decode units.
    const bool tileable = bs == 16 && pd.head_dim == pd.v_head_dim && (pd.head_dim == 64 || pd.head_dim == 128);

    // Pass 1: validate rows (the reference's throws, PagedAttentionKernel.cs:34-39,
    // plus the table and pool bounds) and size the packed arrays.
    int64_t total_q = 0, packed_pages = 0, kv_tokens = 0, pair_pages = 0, max_pages = 0;
    int32_t max_id = -1;  // largest pool block id the step reads
    bool any_tiles = false;
    if (desc->n_bt_ids < 0) return fail(GSP_E_INVALID_ARG, "n_bt_ids must be >= 0 (got %d)", desc->n_bt_ids);
    // The CSR must stay inside the caller's id array: every row span is read
    // through bt_offsets, so they are checked before any id is.
    for (int32_t b = 0; b < B; ++b) {
        const int32_t o0 = desc->bt_offsets[b], o1 = desc->bt_offsets[b + 1];
        if (o0 < 0 || o1 < o0 || o1 > desc->n_bt_ids)
            return fail(GSP_E_INVALID_ARG, "row %d: bt_offsets [%d, %d) outside [0, n_bt_ids = %d] or decreasing",
                             b, o0, o1, desc->n_bt_ids);
    }
    for (int32_t b = 0; b < B; ++b) {
        const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
        const int32_t pos = desc->positions[b];
        const int32_t tc = desc->token_counts[b];
        if (ql < 0) return fail(GSP_E_INVALID_ARG, "row %d: q_len must be >= 0 (got %d)", b, ql);
        const int64_t last = (int64_t)pos + std::max(ql, 1) - 1;
        if (pos < 0 || last >= L)
            return fail(GSP_E_INVALID_ARG, "row %d: token position %lld exceeds valid sequence range [0, %d]", b,
                             (long long)(pos < 0 ? pos : last), L - 1);
        if (tc < 0) return fail(GSP_E_INVALID_ARG, "row %d: token count %d is negative", b, tc);
        if (tc > L) return fail(GSP_E_INVALID_ARG, "row %d: BlockTable token count %d exceeds maxSeqLen %d", b, tc, L);
        const int32_t span = desc->bt_offsets[b + 1] - desc->bt_offsets[b];
        const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
        const int64_t ppages = (total_last + pbs - 1) / pbs;  // pool pages
        if (ppages > span)
            return fail(GSP_E_INVALID_ARG, "row %d: %lld tokens need %lld blocks but the table holds %d", b,
                             (long long)total_last, (long long)ppages, span);
        const int32_t* ids = desc->bt_ids + desc->bt_offsets[b];
        for (int64_t i = 0; i < ppages; ++i) {
            if (ids[i] < 0 || ids[i] >= pd.total_blocks)
                return fail(GSP_E_INVALID_ARG, "row %d: block id %d out of range [0, %d)", b, ids[i],
                                 pd.total_blocks);
            max_id = std::max(max_id, ids[i]);
        }
        const int64_t pages = (total_last + bs - 1) / bs;  // kernel pages
        total_q += ql;
        packed_pages += pages;
        kv_tokens += total_last;
        if (row_is_tiled(opt.prefill_path, ql, tileable)) {  // tiles, not split-KV units
            any_tiles = any_tiles || tc > 0;
            continue;
        }
        max_pages = std::max(max_pages, (total_last + tt - 1) / tt);
        for (int32_t i = 0; i < ql; ++i) {
            const int64_t tot = std::min<int64_t>(tc, (int64_t)pos + i + 1);
            pair_pages += (tot + tt - 1) / tt;
        }
    }
    if (total_q > INT32_MAX / 4 || packed_pages > INT32_MAX / 4 || pair_pages * H > INT32_MAX / 2)
        return fail(GSP_E_INVALID_ARG, "step too large");
    // From here on the tables are in kernel pages: for pool pages above 16
    // tokens, each row's table is expanded into kernel page ids.  The write
    // slots (pass 3) keep pool blocks and slots.
    const gsp_step_desc* const pdesc = desc;
    gsp_step_desc vdesc;
    if (r > 1) {
        voffs_.resize((size_t)B + 1);
        vids_.resize((size_t)packed_pages);
        int64_t w = 0;
        voffs_[0] = 0;
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
            const int64_t total_last = ql > 0 ? std::min<int64_t>(desc->token_counts[b], (int64_t)desc->positions[b] + ql) : 0;
            const int64_t pages = (total_last + bs - 1) / bs;
            const int32_t* ids = desc->bt_ids + desc->bt_offsets[b];
            for (int64_t k = 0; k < pages; ++k) vids_[(size_t)w++] = (int32_t)(ids[k / r] * vfactor + k % r);
            voffs_[(size_t)b + 1] = (int32_t)w;
        }
        vdesc = *desc;
        vdesc.bt_offsets = voffs_.data();
        vdesc.bt_ids = vids_.data();
        vdesc.n_bt_ids = (int32_t)w;
        desc = &vdesc;
    }

    // Pass 2: split-KV units.  Each query token is cut into nsplit near-equal
    // page ranges of at most `target` pages; a unit is one (query token, KV
    // head, page range) and one workgroup.  Units are sorted longest first, so
    // in-order dispatch schedules them longest-processing-time first.
    const int64_t T = pair_pages * H;
    // A pair is cut into at most kMaxSplits pieces.
    const int64_t min_target = std::max<int64_t>(1, (max_pages + kMaxSplits - 1) / kMaxSplits);
    // Default grid: two workgroups per CU, bins balanced per CU (assign_bins).
    // A step that also has prefill tiles runs them beside the decode units
    // (gsp_attention_step): the HBM-bound decode grid then takes one
    // workgroup per four CUs and leaves the other slots to the matrix-bound
    // tiles, which take several times longer (config 4 measured 428 us this
    // way, against 452 us with one per two CUs and 487 us with one per CU).
    const bool pair_cus = opt.decode_bins_override <= 0 && !any_tiles;
    const int64_t bins_max = opt.decode_bins_override > 0 ? (int64_t)opt.decode_bins_override
                             : pair_cus                    ? (int64_t)kDecodeBinsPerCu * std::max(1, opt.num_cus)
                                                           : (int64_t)std::max(1, opt.num_cus / 4);
    const int64_t sim_bins = pair_cus ? bins_max / kDecodeBinsPerCu : bins_max;
    int64_t target = 1;
    if (T > 0) {
        if (opt.split_pages_override > 0) {
            target = std::max<int64_t>(opt.split_pages_override, min_target);
        } else if (max_pages <= kWholePairMaxPages && T <= kUnderloadPagesPerBin * bins_max) {
            target = std::max<int64_t>(1, max_pages);  // whole pairs
        } else if (cached_target_ > 0 && cached_heads_kv_ == H && cached_queries_ == total_q &&
                   cached_bins_ == bins_max && T * 100 >= cached_tasks_ * 97 &&
                   T * 100 <= cached_tasks_ * 103) {
            target = std::max<int64_t>(cached_target_, min_target);  // engine steps drift slowly
        } else {
            query_pages_.clear();
            for (int32_t b = 0; b < B; ++b) {
                const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
                if (row_is_tiled(opt.prefill_path, ql, tileable)) continue;
                for (int32_t i = 0; i < ql; ++i) {
                    const int64_t tot = std::min<int64_t>(desc->token_counts[b], (int64_t)desc->positions[b] + i + 1);
                    if (tot > 0) query_pages_.push_back((int32_t)((tot + tt - 1) / tt));
                }
            }
            int64_t best_cost = INT64_MAX;
            for (int32_t cand : kSplitCandidates) {
                if (cand < min_target) continue;
                if (T / cand > 16 * bins_max) continue;  // far too many units to be competitive
                const int64_t c = simulate_split(query_pages_, H, cand, sim_bins, sim_count_, sim_heap_);
                if (c <= best_cost) {  // ties go to the larger split (fewer units)
                    best_cost = c;
                    target = cand;
                }
                if (cand >= max_pages) break;  // larger candidates give the same units
            }
            cached_target_ = (int32_t)target;
            cached_tasks_ = T;
            cached_heads_kv_ = H;
            cached_queries_ = total_q;
            cached_bins_ = bins_max;
        }
    }
    units_.clear();
    tiles_.clear();
    split_items_.clear();
    q_ctx_.assign((size_t)total_q, 0);
    // fp32 tiles read split records (one per page pair of each tiled row and
    // KV head) unless the caller asked the tiles to split their own pages.
    const bool records = tileable && pd.kv_dtype == GSP_KV_F32 && opt.prefill_split == GSP_SPLIT_RECORDS;
    int64_t n_records = 0;
    int32_t split_max_pairs = 0;
    // grid.y of the split kernel holds one (row, KV head) each.
    constexpr size_t kMaxSplitItems = 65535;
    int64_t slots = 0, pairs_split = 0, tiled_queries = 0, tiled_pairs = 0;
    {
        int64_t qi = 0, bt_base = 0;
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
            const int32_t pos = desc->positions[b];
            const int32_t tc = desc->token_counts[b];
            const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
            if (row_is_tiled(opt.prefill_path, ql, tileable)) {
                // Causal tiles of 16 query tokens; a row with TokenCount 0 has
                // total 0 for every token and gets none (out left untouched).
                for (int32_t i = 0; i < ql; ++i)
                    q_ctx_[qi + i] = (int32_t)std::min<int64_t>(tc, (int64_t)pos + i + 1);
                if (tc > 0) {
                    // The row's page pairs: every tile of the row reads a prefix of them.
                    const int32_t row_pairs = (int32_t)(((total_last + bs - 1) / bs + 1) / 2);
                    const int64_t rec_row = n_records;
                    if (records) {
                        for (int32_t kvh = 0; kvh < H; ++kvh)
                            split_items_.push_back(PrefillSplitItem{
                                (int32_t)bt_base, (int32_t)total_last, kvh, (int32_t)(rec_row + (int64_t)kvh * row_pairs)});
                        n_records += (int64_t)H * row_pairs;
                        split_max_pairs = std::max(split_max_pairs, row_pairs);
                    }
                    for (int32_t t0 = 0; t0 < ql; t0 += kPrefillTileTokens) {
                        PrefillTile t;
                        t.qi0 = (int32_t)(qi + t0);
                        t.bt_base = (int32_t)bt_base;
                        t.pos0 = pos + t0;
                        t.ntok = std::min(kPrefillTileTokens, ql - t0);
                        t.token_count = tc;
                        const int64_t last = std::min<int64_t>(tc, (int64_t)t.pos0 + t.ntok);
                        t.pages = (int32_t)((last + bs - 1) / bs);
                        for (int32_t kvh = 0; kvh < H; ++kvh) {
                            t.kvh = kvh;
                            t.rec0 = records ? (int32_t)(rec_row + (int64_t)kvh * row_pairs) : 0;
                            tiles_.push_back(t);
                        }
                    }
                    for (int32_t i = 0; i < ql; ++i) tiled_pairs += q_ctx_[qi + i];
                    tiled_queries += ql;
                }
                qi += ql;
                bt_base += (total_last + bs - 1) / bs;
                continue;
            }
            for (int32_t i = 0; i < ql; ++i, ++qi) {
                const int32_t tot = (int32_t)std::min<int64_t>(tc, (int64_t)pos + i + 1);
                q_ctx_[qi] = tot;
                if (tot <= 0) continue;
                const int32_t pages = (int32_t)(((int64_t)tot + tt - 1) / tt);  // tiles
                const int32_t nsplit = (int32_t)std::min<int64_t>((pages + target - 1) / target, kMaxSplits);
                const int32_t base = pages / nsplit, extra = pages % nsplit;
                for (int32_t kvh = 0; kvh < H; ++kvh) {
                    for (int32_t s = 0; s < nsplit; ++s) {
                        DecodeUnit u;
                        u.qi = (int32_t)qi;
                        u.bt_base = (int32_t)bt_base;
                        u.page_begin = s * base + std::min(s, extra);
                        u.page_end = u.page_begin + base + (s < extra ? 1 : 0);
                        u.ctx = tot;
                        u.kvh = kvh;
                        u.slot = nsplit > 1 ? (int32_t)slots : -1;
                        u.split_info = s | (nsplit << 16);
                        const int32_t* row_ids = desc->bt_ids + desc->bt_offsets[b];
                        // Each wave's first two tiles: their (first) pages' blocks.
                        for (int w = 0; w < kDecodeWaves; ++w) {
                            const int32_t p = u.page_begin + w;
                            const int32_t p2 = p + kDecodeWaves;
                            u.first_blk[w] = p < u.page_end ? row_ids[(int64_t)p * m] : -1;
                            u.second_blk[w] = p2 < u.page_end ? row_ids[(int64_t)p2 * m] : -1;
                        }
                        units_.push_back(u);
                    }
                    if (nsplit > 1) {
                        slots += nsplit;
                        ++pairs_split;
                    }
                }
            }
            bt_base += (total_last + bs - 1) / bs;
        }
    }
    // Longest first, ties in build order: a counting sort of unit indices by
    // page count (the records themselves move once, into the step image).
    {
        int32_t max_len = 0;
        for (const DecodeUnit& u : units_) max_len = std::max(max_len, u.page_end - u.page_begin);
        auto& cnt = len_count_;
        cnt.assign((size_t)max_len + 2, 0);
        for (const DecodeUnit& u : units_) cnt[(size_t)(max_len - (u.page_end - u.page_begin)) + 1] += 1;
        for (size_t l = 1; l < cnt.size(); ++l) cnt[l] += cnt[l - 1];
        unit_order_.resize(units_.size());
        for (size_t i = 0; i < units_.size(); ++i) {
            const DecodeUnit& u = units_[i];
            unit_order_[(size_t)cnt[(size_t)(max_len - (u.page_end - u.page_begin))]++] = (int32_t)i;
        }
    }
    if (split_items_.size() > kMaxSplitItems) {  // the tiles split their own pages
        split_items_.clear();
        n_records = 0;
        split_max_pairs = 0;
    }
    std::stable_sort(tiles_.begin(), tiles_.end(),
                     [](const PrefillTile& x, const PrefillTile& y) { return x.pages > y.pages; });
    const int32_t n_bins = assign_bins(bins_max, pair_cus);

    // Pass 3: write the staging buffer and upload it with one copy.
    const size_t n_units = units_.size();
    const size_t n_tiles = tiles_.size();
    size_t off = kHdrWords;
    const size_t off_rows = off;
    off += (size_t)B + 1;
    const size_t off_ids = off;
    off += (size_t)packed_pages;
    const size_t off_ctx = off;
    off += (size_t)total_q;
    // Where each query token's own K/V goes (gsp_*_write_step): its position,
    // and the block and slot of that position, or block -1 without a slot.
    const size_t off_wr = off;
    off += 3 * (size_t)total_q;
    off = align_up(off, 8);
    const size_t off_units = off;
    off += n_units * (sizeof(DecodeUnit) / sizeof(int32_t));
    const size_t off_tiles = off;
    off += n_tiles * (sizeof(PrefillTile) / sizeof(int32_t));
    const size_t n_split = split_items_.size();
    const size_t off_split = off;
    off += n_split * (sizeof(PrefillSplitItem) / sizeof(int32_t));
    const size_t off_bins = off;
    off += (size_t)n_bins + 1;
    const size_t words = off;

    // The step image is written in cached host memory; gsp_step_pack copies it
    // into the pinned slot in one pass (element-wise stores straight into the
    // pinned buffer measured several times slower).
    out.image.resize(words);
    int32_t* st = out.image.data();
    std::memset(st, 0, kHdrWords * sizeof(int32_t));
    {
        int32_t* rows = st + off_rows;
        int32_t* ids = st + off_ids;
        int32_t* wr_pos = st + off_wr;
        int32_t* wr_blk = wr_pos + total_q;
        int32_t* wr_slot = wr_blk + total_q;
        int64_t w = 0, qi = 0;
        rows[0] = 0;
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
            const int32_t pos = desc->positions[b];
            const int32_t tc = desc->token_counts[b];
            const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
            const int64_t pages = (total_last + bs - 1) / bs;
            const int32_t* src = desc->bt_ids + desc->bt_offsets[b];
            const int32_t* psrc = pdesc->bt_ids + pdesc->bt_offsets[b];  // pool blocks
            for (int64_t i = 0; i < pages; ++i) ids[w++] = src[i];
            rows[b + 1] = (int32_t)w;
            // A query token at p < TokenCount has its slot in the packed pages
            // (p < total_last); the reference stores its K/V there before
            // attending (PagedTransformerRunner.cs:620-634, :437-452).
            for (int32_t i = 0; i < ql; ++i, ++qi) {
                const int64_t p = (int64_t)pos + i;
                wr_pos[qi] = (int32_t)p;
                const bool has = p < tc;
                wr_blk[qi] = has ? psrc[p / pbs] : -1;
                wr_slot[qi] = has ? (int32_t)(p % pbs) : 0;
            }
        }
    }
    if (total_q) std::memcpy(st + off_ctx, q_ctx_.data(), (size_t)total_q * sizeof(int32_t));
    {
        DecodeUnit* dst = reinterpret_cast<DecodeUnit*>(st + off_units);
        for (size_t j = 0; j < n_units; ++j) dst[j] = units_[(size_t)unit_place_[j]];
    }
    if (n_tiles) std::memcpy(st + off_tiles, tiles_.data(), n_tiles * sizeof(PrefillTile));
    if (n_split) std::memcpy(st + off_split, split_items_.data(), n_split * sizeof(PrefillSplitItem));
    std::memcpy(st + off_bins, bin_units_.data(), ((size_t)n_bins + 1) * sizeof(int32_t));
    st[kHdrRows] = B;
    st[kHdrTotalQ] = (int32_t)total_q;
    st[kHdrPages] = (int32_t)packed_pages;
    st[kHdrUnits] = (int32_t)n_units;
    st[kHdrTarget] = (int32_t)target;
    st[kHdrSlots] = (int32_t)slots;
    st[kHdrMaxId] = max_id;
    st[kHdrPairsSplit] = (int32_t)pairs_split;
    st[kHdrHeadsKv] = H;
    st[kHdrTiles] = (int32_t)n_tiles;
    st[kHdrBins] = n_bins;

    out.off_rows = off_rows;
    out.off_ids = off_ids;
    out.off_ctx = off_ctx;
    out.off_wr = off_wr;
    out.off_units = off_units;
    out.off_tiles = off_tiles;
    out.off_split = off_split;
    out.off_bins = off_bins;
    out.num_rows = B;
    out.total_q = total_q;
    out.packed_pages = packed_pages;
    out.kv_tokens = kv_tokens;
    out.num_units = (int32_t)n_units;
    out.num_bins = n_bins;
    out.num_tiles = (int32_t)n_tiles;
    out.num_slots = slots;
    out.pairs_split = pairs_split;
    out.target = (int32_t)target;
    out.num_split_items = (int32_t)n_split;
    out.split_max_pairs = split_max_pairs;
    out.num_records = n_records;
    out.tiled_queries = tiled_queries;
    out.tiled_pairs = tiled_pairs;
    out.max_id = max_id;
    out.tileable = tileable;
    out.page_tokens = bs;
    out.tile_pages = m;
    out.pool_page_split = r;
    return GSP_OK;
}

}  // namespace gsp
