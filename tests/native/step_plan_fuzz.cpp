// Drives the host step packer (gsp_step_plan.cpp) without a GPU, built with
// AddressSanitizer + UndefinedBehaviorSanitizer by the Makefile beside it.
//
//   step_plan_fuzz STEPS_FILE
//
// STEPS_FILE holds valid engine steps (the five measured shapes and smaller
// ones, written by tests/test_step_plan_native.py).  For each step:
//  1. it is planned with the default options and with forced split sizes, bin
//     counts and prefill routes; each plan must succeed and its image must
//     hold the packed tables, every unit's pages exactly once per (query, KV
//     head), consistent split slots, bins that cover every unit once, and
//     tiles and write slots inside their rows;
//  2. seeded malformed copies of it (CSR offsets out of order or out of
//     range, short tables, block ids outside the pool, positions and token
//     counts outside [0, maxSeqLen), negative or huge query lengths, NULL
//     arrays) must each be refused with GSP_E_INVALID_ARG.
// Then random steps over wide value ranges must either be refused with
// GSP_E_INVALID_ARG or plan into an image that passes the same checks.
// Exit status 0 when everything held; the sanitizers abort on their own.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "gsp_step_plan.h"

namespace {

struct Step {
    gsp::PlanPool pool;
    int32_t max_seq_len = 0;
    bool has_qlens = false;
    std::vector<int32_t> positions, q_lens, token_counts, offsets, ids;
    int32_t rows() const { return (int32_t)positions.size(); }
    int32_t ql(int32_t b) const { return has_qlens ? q_lens[(size_t)b] : 1; }
};

int g_failures = 0;

void failf(const char* what, const std::string& ctx) {
    std::fprintf(stderr, "FAIL %s: %s\n", ctx.c_str(), what);
    ++g_failures;
}

bool read_steps(const char* path, std::vector<Step>& out) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    auto rd = [&](int32_t* p, size_t n) { return n == 0 || std::fread(p, sizeof(int32_t), n, f) == n; };
    int32_t magic = 0, count = 0;
    if (!rd(&magic, 1) || magic != 0x53505347 || !rd(&count, 1)) return false;
    for (int32_t s = 0; s < count; ++s) {
        int32_t h[11];
        if (!rd(h, 11)) return false;
        Step st;
        st.pool.total_blocks = h[0];
        st.pool.heads_kv = h[1];
        st.pool.head_dim = h[2];
        st.pool.v_head_dim = h[3];
        st.pool.block_size = h[4];
        st.pool.kv_dtype = h[5];
        const int32_t B = h[6];
        st.max_seq_len = h[7];
        st.has_qlens = h[8] != 0;
        const int32_t n_ids = h[9];
        st.pool.layers = h[10];
        st.positions.resize((size_t)B);
        st.token_counts.resize((size_t)B);
        st.offsets.resize((size_t)B + 1);
        st.ids.resize((size_t)n_ids);
        if (st.has_qlens) st.q_lens.resize((size_t)B);
        if (!rd(st.positions.data(), (size_t)B) || (st.has_qlens && !rd(st.q_lens.data(), (size_t)B)) ||
            !rd(st.token_counts.data(), (size_t)B) || !rd(st.offsets.data(), (size_t)B + 1) ||
            !rd(st.ids.data(), (size_t)n_ids))
            return false;
        out.push_back(std::move(st));
    }
    std::fclose(f);
    return true;
}

gsp_step_desc make_desc(const Step& st) {
    gsp_step_desc d;
    d.num_rows = st.rows();
    d.max_seq_len = st.max_seq_len;
    d.positions = st.positions.data();
    d.q_lens = st.has_qlens ? st.q_lens.data() : nullptr;
    d.token_counts = st.token_counts.data();
    d.bt_offsets = st.offsets.data();
    d.bt_ids = st.ids.data();
    d.n_bt_ids = (int32_t)st.ids.size();
    return d;
}

// Checks a successful plan's image against the step it came from.
void check_image(const Step& st, const gsp::StepPlan& p, const std::string& ctx) {
    const int32_t* im = p.image.data();
    const size_t words = p.image.size();
    const int32_t B = st.rows();
    const int32_t pbs = st.pool.block_size;  // pool page
    int32_t bs = std::min(pbs, 16);          // kernel page: the largest divisor of pbs up to 16
    while (pbs % bs) --bs;
    const int32_t r = pbs / bs;
    const int32_t H = st.pool.heads_kv;
    if (p.page_tokens != bs || p.pool_page_split != r) return failf("kernel page size", ctx);
    // Decode units count tiles of m pages (4- and 8-token pages: 16 tokens).
    const int32_t m = (r == 1 && (bs == 4 || bs == 8)) ? 16 / bs : 1;
    const int32_t tt = bs * m;
    if (p.tile_pages != m) return failf("tile pages", ctx);
    // Kernel page k of a row: sub-page k % r of pool page k / r.
    auto kernel_id = [&](int32_t b, int64_t k) -> int64_t {
        const int64_t blk = st.ids[(size_t)st.offsets[(size_t)b] + (size_t)(k / r)];
        return r == 1 ? blk : blk * ((int64_t)st.pool.layers * H * r) + k % r;
    };
    auto in_image = [&](size_t off, size_t n) { return off <= words && n <= words - off; };
    if (!in_image(0, gsp::kHdrWords) || im[gsp::kHdrRows] != B || im[gsp::kHdrUnits] != p.num_units ||
        im[gsp::kHdrTiles] != p.num_tiles || im[gsp::kHdrBins] != p.num_bins || im[gsp::kHdrHeadsKv] != H ||
        (int64_t)im[gsp::kHdrTotalQ] != p.total_q)
        return failf("header", ctx);
    if (!in_image(p.off_rows, (size_t)B + 1) || !in_image(p.off_ids, (size_t)p.packed_pages) ||
        !in_image(p.off_ctx, (size_t)p.total_q) || !in_image(p.off_wr, 3 * (size_t)p.total_q) ||
        !in_image(p.off_units, (size_t)p.num_units * 16) || !in_image(p.off_tiles, (size_t)p.num_tiles * 8) ||
        !in_image(p.off_split, (size_t)p.num_split_items * 4) || !in_image(p.off_bins, (size_t)p.num_bins + 1))
        return failf("array outside the image", ctx);
    // Packed tables: each row's span cut to ceil(total / bs).
    const int32_t* rows = im + p.off_rows;
    const int32_t* ids = im + p.off_ids;
    std::vector<int64_t> row_pages((size_t)B), row_first_q((size_t)B);
    int64_t q = 0;
    if (rows[0] != 0) return failf("row_offsets[0]", ctx);
    for (int32_t b = 0; b < B; ++b) {
        const int64_t ql = st.ql(b);
        const int64_t tot = ql > 0 ? std::min<int64_t>(st.token_counts[(size_t)b], (int64_t)st.positions[(size_t)b] + ql) : 0;
        const int64_t pages = (tot + bs - 1) / bs;
        row_pages[(size_t)b] = pages;
        row_first_q[(size_t)b] = q;
        q += ql;
        if (rows[b + 1] - rows[b] != pages) return failf("row span", ctx);
        for (int64_t i = 0; i < pages; ++i)
            if (ids[rows[b] + i] != kernel_id(b, i)) return failf("packed id", ctx);
    }
    if (q != p.total_q) return failf("total_q", ctx);
    // Write slots.
    const int32_t* wr_pos = im + p.off_wr;
    const int32_t* wr_blk = wr_pos + p.total_q;
    const int32_t* wr_slot = wr_blk + p.total_q;
    for (int32_t b = 0; b < B; ++b)
        for (int32_t i = 0; i < st.ql(b); ++i) {
            const int64_t qi = row_first_q[(size_t)b] + i;
            const int64_t pos = (int64_t)st.positions[(size_t)b] + i;
            if (wr_pos[qi] != pos) return failf("write position", ctx);
            const bool has = pos < st.token_counts[(size_t)b];
            const int32_t pool_blk = has ? st.ids[(size_t)st.offsets[(size_t)b] + (size_t)(pos / pbs)] : -1;
            if (has ? (wr_blk[qi] != pool_blk || wr_slot[qi] != pos % pbs) : wr_blk[qi] != -1)
                return failf("write slot", ctx);
        }
    // Units: pages of each (query, KV head) covered once; splits consistent.
    const gsp::DecodeUnit* units = reinterpret_cast<const gsp::DecodeUnit*>(im + p.off_units);
    std::vector<int32_t> q_of_row((size_t)p.total_q, -1);
    for (int32_t b = 0; b < B; ++b)
        for (int32_t i = 0; i < st.ql(b); ++i) q_of_row[(size_t)(row_first_q[(size_t)b] + i)] = b;
    std::vector<int64_t> covered((size_t)p.total_q * (size_t)H, 0);
    std::vector<int32_t> seen_slots((size_t)std::max<int64_t>(p.num_slots, 0), 0);
    for (int32_t j = 0; j < p.num_units; ++j) {
        const gsp::DecodeUnit& u = units[j];
        if (u.qi < 0 || u.qi >= p.total_q || u.kvh < 0 || u.kvh >= H) return failf("unit query/head", ctx);
        const int32_t b = q_of_row[(size_t)u.qi];
        const int64_t pos = (int64_t)st.positions[(size_t)b] + (u.qi - row_first_q[(size_t)b]);
        const int64_t tot = std::min<int64_t>(st.token_counts[(size_t)b], pos + 1);
        const int64_t pages = (tot + tt - 1) / tt;  // tiles
        if (u.ctx != tot || u.bt_base != rows[b] || u.page_begin < 0 || u.page_end > pages ||
            u.page_begin >= u.page_end)
            return failf("unit range", ctx);
        for (int w = 0; w < gsp::kDecodeWaves; ++w) {
            const int32_t p1 = u.page_begin + w, p2 = p1 + gsp::kDecodeWaves;
            if (u.first_blk[w] != (p1 < u.page_end ? ids[rows[b] + (int64_t)p1 * m] : -1) ||
                u.second_blk[w] != (p2 < u.page_end ? ids[rows[b] + (int64_t)p2 * m] : -1))
                return failf("unit block ids", ctx);
        }
        covered[(size_t)u.qi * (size_t)H + (size_t)u.kvh] += u.page_end - u.page_begin;
        const int32_t nsplit = u.split_info >> 16, split = u.split_info & 0xFFFF;
        if (nsplit < 1 || split >= nsplit) return failf("split info", ctx);
        if (nsplit == 1 ? u.slot != -1 : (u.slot < 0 || (int64_t)u.slot + nsplit > p.num_slots))
            return failf("split slot", ctx);
        if (nsplit > 1 && seen_slots[(size_t)(u.slot + split)]++) return failf("split slot used twice", ctx);
    }
    // Every query token of a row without tiles has its pages covered exactly
    // once per KV head by its units; a tiled row has no units.
    std::vector<char> tiled((size_t)B, 0);
    {
        const gsp::PrefillTile* tl = reinterpret_cast<const gsp::PrefillTile*>(im + p.off_tiles);
        for (int32_t j = 0; j < p.num_tiles; ++j)
            if (tl[j].qi0 >= 0 && tl[j].qi0 < p.total_q) tiled[(size_t)q_of_row[(size_t)tl[j].qi0]] = 1;
    }
    for (int64_t qi = 0; qi < p.total_q; ++qi) {
        const int32_t b = q_of_row[(size_t)qi];
        const int64_t pos = (int64_t)st.positions[(size_t)b] + (qi - row_first_q[(size_t)b]);
        const int64_t tot = std::min<int64_t>(st.token_counts[(size_t)b], pos + 1);
        const int64_t want = tiled[(size_t)b] || tot <= 0 ? 0 : (tot + tt - 1) / tt;
        for (int32_t h = 0; h < H; ++h)
            if (covered[(size_t)qi * (size_t)H + (size_t)h] != want) return failf("unit coverage", ctx);
    }
    // Bins: bin_rest[0] == num_bins, monotone, covering every unit once.
    const int32_t* bins = im + p.off_bins;
    if (p.num_units > 0 && (bins[0] != p.num_bins || bins[p.num_bins] != p.num_units)) return failf("bin ends", ctx);
    for (int32_t k = 0; k < p.num_bins; ++k)
        if (bins[k + 1] < bins[k]) return failf("bin order", ctx);
    // Tiles.
    const gsp::PrefillTile* tiles = reinterpret_cast<const gsp::PrefillTile*>(im + p.off_tiles);
    for (int32_t j = 0; j < p.num_tiles; ++j) {
        const gsp::PrefillTile& t = tiles[j];
        if (t.qi0 < 0 || t.ntok < 1 || t.ntok > gsp::kPrefillTileTokens || (int64_t)t.qi0 + t.ntok > p.total_q ||
            t.kvh < 0 || t.kvh >= H)
            return failf("tile", ctx);
        const int32_t b = q_of_row[(size_t)t.qi0];
        if (t.bt_base != rows[b] || t.pages > row_pages[(size_t)b] || t.pages < 1) return failf("tile pages", ctx);
    }
}

int plan_step(gsp::StepPlanner& planner, const Step& st, const gsp::PlanOptions& opt, gsp::StepPlan& out) {
    const gsp_step_desc d = make_desc(st);
    return planner.plan(st.pool, &d, opt, out);
}

void check_valid(gsp::StepPlanner& planner, const Step& st, int idx) {
    struct Variant {
        int32_t split_pages, bins, path, split;
    };
    const Variant vars[] = {{0, 0, GSP_PREFILL_AUTO, GSP_SPLIT_RECORDS}, {1, 0, GSP_PREFILL_AUTO, GSP_SPLIT_RECORDS},
                            {3, 7, GSP_PREFILL_TILES, GSP_SPLIT_IN_TILE}, {0, 1, GSP_PREFILL_PER_TOKEN, GSP_SPLIT_RECORDS},
                            {48, 1000, GSP_PREFILL_AUTO, GSP_SPLIT_RECORDS}};
    gsp::StepPlan out;
    for (const Variant& v : vars) {
        gsp::PlanOptions opt;
        opt.num_cus = 256;
        opt.split_pages_override = v.split_pages;
        opt.decode_bins_override = v.bins;
        opt.prefill_path = v.path;
        opt.prefill_split = v.split;
        const std::string ctx = "step " + std::to_string(idx) + " split " + std::to_string(v.split_pages) + " bins " +
                                std::to_string(v.bins) + " path " + std::to_string(v.path);
        const int rc = plan_step(planner, st, opt, out);
        if (rc != GSP_OK) {
            failf("valid step refused", ctx);
            continue;
        }
        check_image(st, out, ctx);
    }
}

// Seeded malformed copies of a valid step: each must be refused.
void check_malformed(gsp::StepPlanner& planner, const Step& base, int idx, std::mt19937& rng) {
    const int32_t B = base.rows();
    if (B == 0) return;
    gsp::PlanOptions opt;
    opt.num_cus = 256;
    gsp::StepPlan out;
    auto pick = [&](int32_t n) { return (int32_t)(rng() % (uint32_t)n); };
    auto expect_refused = [&](const Step& st, const char* what, const gsp_step_desc* override_desc = nullptr) {
        const gsp_step_desc d = override_desc ? *override_desc : make_desc(st);
        const int rc = planner.plan(st.pool, &d, opt, out);
        if (rc != GSP_E_INVALID_ARG) failf(what, "malformed step " + std::to_string(idx) + " rc " + std::to_string(rc));
    };
    // A row whose packed range is non-empty (for id and short-table cases).
    int32_t rb = -1;
    for (int32_t t = 0; t < 8 * B && rb < 0; ++t) {
        const int32_t b = pick(B);
        const int64_t ql = base.ql(b);
        if (ql > 0 && std::min<int64_t>(base.token_counts[(size_t)b], (int64_t)base.positions[(size_t)b] + ql) > 0) rb = b;
    }
    {
        Step st = base;  // offsets out of order
        const int32_t b = pick(B);
        if (st.offsets[(size_t)b + 1] > st.offsets[(size_t)b]) {
            std::swap(st.offsets[(size_t)b], st.offsets[(size_t)b + 1]);
            expect_refused(st, "decreasing offsets");
        }
    }
    {
        Step st = base;  // an offset past the id array
        st.offsets[(size_t)B] = (int32_t)st.ids.size() + 1 + pick(1000);
        expect_refused(st, "offset past n_bt_ids");
    }
    {
        Step st = base;  // a negative offset
        st.offsets[0] = -1 - pick(1000);
        expect_refused(st, "negative offset");
    }
    if (rb >= 0) {
        Step st = base;  // the id array shorter than the CSR says
        gsp_step_desc d = make_desc(st);
        d.n_bt_ids = st.offsets[(size_t)rb + 1] - 1;
        if (d.n_bt_ids >= 0) expect_refused(st, "n_bt_ids short", &d);
    }
    if (rb >= 0) {
        Step st = base;  // a block id outside the pool
        st.ids[(size_t)st.offsets[(size_t)rb]] = pick(2) ? st.pool.total_blocks + pick(100) : -1 - pick(100);
        expect_refused(st, "block id out of range");
    }
    {
        Step st = base;  // a table shorter than its row's tokens
        const int32_t b = pick(B);
        const int32_t span = st.offsets[(size_t)b + 1] - st.offsets[(size_t)b];
        const int64_t tc = (int64_t)span * st.pool.block_size + 1;
        if (tc <= st.max_seq_len) {
            st.token_counts[(size_t)b] = (int32_t)tc;
            st.positions[(size_t)b] = (int32_t)tc - 1;
            if (st.has_qlens) st.q_lens[(size_t)b] = 1;
            expect_refused(st, "table shorter than tokens");
        }
    }
    {
        Step st = base;  // positions outside [0, maxSeqLen)
        const int32_t b = pick(B);
        st.positions[(size_t)b] = pick(2) ? -1 - pick(100) : st.max_seq_len + pick(100);
        expect_refused(st, "position out of range");
    }
    {
        Step st = base;  // token counts outside [0, maxSeqLen]
        const int32_t b = pick(B);
        st.token_counts[(size_t)b] = pick(2) ? -1 - pick(100) : st.max_seq_len + 1 + pick(100);
        expect_refused(st, "token count out of range");
    }
    {
        Step st = base;  // a negative or huge query length
        if (!st.has_qlens) {
            st.has_qlens = true;
            st.q_lens.assign((size_t)B, 1);
        }
        const int32_t b = pick(B);
        st.q_lens[(size_t)b] = pick(2) ? -1 - pick(100) : (int32_t)(0x7fffffff - pick(100));
        expect_refused(st, "query length out of range");
    }
    {
        Step st = base;  // NULL arrays, bad counts
        gsp_step_desc d = make_desc(st);
        d.positions = nullptr;
        expect_refused(st, "NULL positions", &d);
        d = make_desc(st);
        d.bt_ids = nullptr;
        expect_refused(st, "NULL ids", &d);
        d = make_desc(st);
        d.num_rows = -1 - pick(10);
        expect_refused(st, "negative rows", &d);
        d = make_desc(st);
        d.max_seq_len = -pick(10);
        expect_refused(st, "maxSeqLen <= 0", &d);
        d = make_desc(st);
        d.n_bt_ids = -1 - pick(10);
        expect_refused(st, "negative n_bt_ids", &d);
    }
}

// Random steps over wide ranges: refused, or planned into a valid image.
void fuzz(gsp::StepPlanner& planner, std::mt19937& rng, int iters) {
    gsp::StepPlan out;
    int accepted = 0;
    for (int it = 0; it < iters; ++it) {
        auto u = [&](int64_t lo, int64_t hi) { return (int32_t)(lo + (int64_t)(rng() % (uint64_t)(hi - lo + 1))); };
        Step st;
        st.pool.block_size = u(0, 3) ? u(1, 16) : u(17, 64);
        st.pool.layers = u(1, 4);
        st.pool.heads_kv = u(1, 8);
        st.pool.head_dim = 2 * u(1, 128);
        st.pool.v_head_dim = u(0, 3) ? st.pool.head_dim : 2 * u(1, 128);
        st.pool.kv_dtype = u(0, 1) ? GSP_KV_F16 : GSP_KV_F32;
        st.pool.total_blocks = u(1, 4096);
        // One step in 16 is large: few rows, contexts up to two million tokens
        // near the top of the int32 range of maxSeqLen and positions.
        const bool large = u(0, 15) == 0;
        const int32_t B = large ? u(1, 3) : u(0, 24);
        const int32_t ctx_hi = large ? 2000000 : 3000;
        st.max_seq_len = u(0, 10) == 0 ? u(-4, 4) : (u(0, 20) == 0 || large ? (int32_t)0x7fffffff - u(0, 20) : u(1, 3000));
        st.has_qlens = u(0, 1);
        int64_t off = 0;
        st.offsets.push_back(0);
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = st.has_qlens ? (u(0, 15) == 0 ? u(-3, 3) : (u(0, 3) ? 1 : u(0, 80))) : 1;
            const int32_t tc = u(0, 12) == 0 ? u(-5, 5) : u(0, std::max(0, std::min(st.max_seq_len, ctx_hi)));
            const int32_t pos = u(0, 12) == 0 ? u(-5, st.max_seq_len > 0 ? std::min(st.max_seq_len, ctx_hi + 1000) : 5)
                                : u(0, 20) == 0 ? (int32_t)0x7fffffff - u(0, 40)
                                                : std::max(0, tc - std::max(ql, 1) + u(-2, 2));
            st.positions.push_back(pos);
            if (st.has_qlens) st.q_lens.push_back(ql);
            st.token_counts.push_back(tc);
            const int64_t need = tc > 0 ? ((int64_t)tc + st.pool.block_size - 1) / st.pool.block_size : 0;
            const int64_t span = std::max<int64_t>(0, need + (u(0, 10) == 0 ? u(-2, 2) : 0));
            for (int64_t i = 0; i < span; ++i)
                st.ids.push_back(u(0, 30) == 0 ? u(-3, st.pool.total_blocks + 3) : u(0, st.pool.total_blocks - 1));
            off += span;
            st.offsets.push_back((int32_t)off);
        }
        if (B > 0 && u(0, 15) == 0) st.offsets[(size_t)u(0, B)] += u(-3, 3);
        const gsp_step_desc d = make_desc(st);
        gsp::PlanOptions opt;
        opt.num_cus = u(1, 256);
        opt.split_pages_override = u(0, 3) ? 0 : u(1, 40);
        opt.decode_bins_override = u(0, 3) ? 0 : u(1, 600);
        opt.prefill_path = u(0, 2);
        opt.prefill_split = u(0, 1);
        const int rc = planner.plan(st.pool, &d, opt, out);
        if (rc == GSP_OK) {
            ++accepted;
            check_image(st, out, "fuzz " + std::to_string(it));
        } else if (rc != GSP_E_INVALID_ARG && !(rc == GSP_E_UNSUPPORTED && st.pool.block_size > 16)) {
            failf("unexpected status", "fuzz " + std::to_string(it));
        }
    }
    std::printf("fuzz: %d steps, %d planned, %d refused\n", iters, accepted, iters - accepted);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s STEPS_FILE [FUZZ_ITERS]\n", argv[0]);
        return 2;
    }
    std::vector<Step> steps;
    if (!read_steps(argv[1], steps)) {
        std::fprintf(stderr, "cannot read %s\n", argv[1]);
        return 2;
    }
    const int iters = argc > 2 ? std::atoi(argv[2]) : 3000;
    gsp::StepPlanner planner;
    std::mt19937 rng(20261202u);
    for (size_t i = 0; i < steps.size(); ++i) {
        check_valid(planner, steps[i], (int)i);
        for (int r = 0; r < 8; ++r) check_malformed(planner, steps[i], (int)i, rng);
    }
    std::printf("valid and malformed: %zu steps\n", steps.size());
    fuzz(planner, rng, iters);
    if (g_failures) {
        std::fprintf(stderr, "%d failures\n", g_failures);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
