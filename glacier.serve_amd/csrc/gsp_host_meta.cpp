// Host-side block metadata: the free-stack / refcount half of PagedBlockPool
// (PagedBlockPool.cs:112-121,178-299,332-353), its prefix cache
// (:163-234: the XXH3 hash chain over full blocks' token ids and the map from
// a prefix hash to the block that holds it) and BlockTable
// (BlockTable.cs:13-117).  Pages themselves live in a device pool; an attached
// pool receives the copy-on-write page copies.
#include <algorithm>

#include "gsp_host_meta.h"
#include "gsp_status.h"
#include "gsp_xxh3.h"

extern "C" {

int gsp_block_allocator_create(int32_t total_blocks, int32_t block_size, gsp_block_allocator** out) {
    gsp::clear_error();
    if (!out) return gsp::fail(GSP_E_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (total_blocks < 1) return gsp::fail(GSP_E_INVALID_ARG, "totalBlocks must be >= 1 (got %d)", total_blocks);
    if (block_size < 1) return gsp::fail(GSP_E_INVALID_ARG, "blockSize must be >= 1 (got %d)", block_size);
    gsp_block_allocator* a = new gsp_block_allocator();
    a->total = total_blocks;
    a->block_size = block_size;
    a->allocated.reset(new std::atomic<int32_t>[total_blocks]);
    a->refs.reset(new std::atomic<int32_t>[total_blocks]);
    a->hashes.reset(new std::atomic<uint64_t>[total_blocks]);
    a->free_stack.reserve(total_blocks);
    // Pushing total-1 .. 0 leaves 0 on top: the first pop returns block 0.
    for (int32_t i = total_blocks - 1; i >= 0; --i) {
        a->allocated[i].store(0);
        a->refs[i].store(0);
        a->hashes[i].store(0);
        a->free_stack.push_back(i);
    }
    *out = a;
    return GSP_OK;
}

void gsp_block_allocator_destroy(gsp_block_allocator* a) { delete a; }

int gsp_block_allocator_try_allocate(gsp_block_allocator* a, int32_t* block_id) {
    gsp::clear_error();
    if (!a || !block_id) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument"), 0;
    return a->try_allocate(block_id) ? 1 : 0;
}

int gsp_block_allocator_retain(gsp_block_allocator* a, int32_t block_id) {
    gsp::clear_error();
    if (!a) return gsp::fail(GSP_E_INVALID_ARG, "allocator is NULL"), -1;
    if (block_id < 0 || block_id >= a->total) {
        gsp::fail(GSP_E_INVALID_ARG, "physicalBlockId %d out of range [0, %d)", block_id, a->total);
        return -1;
    }
    return a->refs[block_id].fetch_add(1) + 1;
}

int gsp_block_allocator_release(gsp_block_allocator* a, int32_t block_id) {
    gsp::clear_error();
    if (!a) return 0;
    return a->release(block_id);
}

int gsp_block_allocator_ref_count(const gsp_block_allocator* a, int32_t block_id) {
    if (!a || block_id < 0 || block_id >= a->total) return 0;
    return a->refs[block_id].load();
}

int gsp_block_allocator_free_count(const gsp_block_allocator* a) {
    if (!a) return 0;
    std::lock_guard<std::mutex> lk(const_cast<gsp_block_allocator*>(a)->stack_mu);
    return (int)a->free_stack.size();
}

int gsp_block_allocator_total(const gsp_block_allocator* a) { return a ? a->total : 0; }

uint64_t gsp_prefix_hash(uint64_t parent_hash, const int32_t* tokens, int32_t n) {
    gsp::clear_error();
    if (n < 0 || (n > 0 && !tokens)) {
        gsp::fail(GSP_E_INVALID_ARG, "token span is invalid");
        return 0;
    }
    // The token ids' bytes as stored (little-endian int32), seeded with the parent.
    return gsp::xxh3::hash64(tokens, (size_t)n * sizeof(int32_t), parent_hash);
}

int gsp_prefix_hash_chain(uint64_t parent_hash, const int32_t* tokens, int32_t n_blocks, int32_t block_size,
                          uint64_t* out) {
    gsp::clear_error();
    if (n_blocks < 0 || block_size < 1 || (n_blocks > 0 && (!tokens || !out)))
        return gsp::fail(GSP_E_INVALID_ARG, "token blocks or output are invalid");
    uint64_t h = parent_hash;
    for (int32_t b = 0; b < n_blocks; ++b) {
        h = gsp::xxh3::hash64(tokens + (int64_t)b * block_size, (size_t)block_size * sizeof(int32_t), h);
        out[b] = h;
    }
    return GSP_OK;
}

int gsp_block_allocator_find_prefix(gsp_block_allocator* a, uint64_t prefix_hash, int32_t* block_id) {
    gsp::clear_error();
    if (!a || !block_id) return gsp::fail(GSP_E_INVALID_ARG, "allocator/block_id is NULL"), 0;
    *block_id = -1;
    if (prefix_hash == 0) return 0;
    int32_t b;
    {
        std::lock_guard<std::mutex> lk(a->map_mu);
        const auto it = a->prefix_map.find(prefix_hash);
        if (it == a->prefix_map.end()) return 0;
        b = it->second;
    }
    // Take a reference only while the block is live, then check that it still
    // holds this prefix (it may have been freed and reused meanwhile).
    int32_t cur = a->refs[b].load();
    while (true) {
        if (cur <= 0) return 0;
        if (a->refs[b].compare_exchange_weak(cur, cur + 1)) break;
    }
    if (a->hashes[b].load() != prefix_hash) {
        a->release(b);
        return 0;
    }
    *block_id = b;
    return 1;
}

int gsp_block_allocator_bind_prefix(gsp_block_allocator* a, uint64_t prefix_hash, int32_t block_id) {
    gsp::clear_error();
    if (!a) return gsp::fail(GSP_E_INVALID_ARG, "allocator is NULL");
    if (block_id < 0 || block_id >= a->total)
        return gsp::fail(GSP_E_INVALID_ARG, "physicalBlockId %d out of range [0, %d)", block_id, a->total);
    if (prefix_hash == 0) return gsp::fail(GSP_E_INVALID_ARG, "Prefix hash cannot be 0.");
    a->hashes[block_id].store(prefix_hash);
    std::lock_guard<std::mutex> lk(a->map_mu);
    a->prefix_map[prefix_hash] = block_id;
    return GSP_OK;
}

int gsp_block_table_create(gsp_block_allocator* a, gsp_block_table** out) {
    gsp::clear_error();
    if (!a || !out) return gsp::fail(GSP_E_INVALID_ARG, "pool/out is NULL");
    gsp_block_table* t = new gsp_block_table();
    t->alloc = a;
    t->ids.reserve(16);
    *out = t;
    return GSP_OK;
}

void gsp_block_table_destroy(gsp_block_table* t) { delete t; }

int gsp_block_table_attach_prefix(gsp_block_table* t, const int32_t* ids, int32_t n, int32_t token_count) {
    gsp::clear_error();
    if (!t) return gsp::fail(GSP_E_INVALID_ARG, "table is NULL");
    if (token_count < 0) return gsp::fail(GSP_E_INVALID_ARG, "tokenCount must be >= 0 (got %d)", token_count);
    if (n < 0 || (n > 0 && !ids)) return gsp::fail(GSP_E_INVALID_ARG, "prefix span is invalid");
    t->ids.insert(t->ids.end(), ids, ids + n);
    t->token_count = token_count;
    return GSP_OK;
}

int gsp_block_table_append_token(gsp_block_table* t, int32_t* block_id, int32_t* offset) {
    gsp::clear_error();
    if (!t || !block_id || !offset) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument"), -1;
    gsp_block_allocator* a = t->alloc;
    const int32_t bs = a->block_size;
    if (t->token_count % bs == 0) {
        int32_t nb;
        if (!a->try_allocate(&nb)) {
            *block_id = -1;
            *offset = -1;
            return 0;
        }
        t->ids.push_back(nb);
    } else {
        // A partial last page that the table does not hold (a prefix attached
        // with fewer ids than its token count needs none, but an empty one
        // has no last page): the reference's _physicalBlockIds[^1] throws.
        if (t->ids.empty()) {
            *block_id = -1;
            *offset = -1;
            return gsp::fail(GSP_E_INVALID_ARG, "tokenCount %d is inside a page but the table holds no pages",
                             t->token_count),
                   -1;
        }
        const int32_t last = t->ids.back();
        if (gsp_block_allocator_ref_count(a, last) > 1) {
            // Copy-on-write fork of a shared partial page (BlockTable.cs:60-73).
            const int32_t in_block = t->token_count % bs;
            int32_t forked;
            if (!a->try_allocate(&forked)) {
                *block_id = -1;
                *offset = -1;
                return 0;
            }
            if (a->copy_page) {
                int rc = a->copy_page(a->ctx, a->pool, last, forked, in_block);
                if (rc) {
                    a->release(forked);
                    *block_id = -1;
                    *offset = -1;
                    return 0;
                }
            }
            a->release(last);
            t->ids.back() = forked;
        }
    }
    *block_id = t->ids.back();
    *offset = t->token_count % bs;
    t->token_count++;
    return 1;
}

int gsp_block_table_append_tokens(gsp_block_table* t, int32_t n) {
    gsp::clear_error();
    if (!t) return gsp::fail(GSP_E_INVALID_ARG, "table is NULL"), 0;
    int32_t b, o, done = 0;
    while (done < n && gsp_block_table_append_token(t, &b, &o) == 1) ++done;
    return done;
}

int gsp_block_table_token_location(const gsp_block_table* t, int32_t token, int32_t* block_id, int32_t* offset) {
    gsp::clear_error();
    if (!t || !block_id || !offset) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    const int32_t bs = t->alloc->block_size;
    const int32_t idx = token < 0 ? -1 : token / bs;
    if (idx < 0 || idx >= (int32_t)t->ids.size())
        return gsp::fail(GSP_E_INVALID_ARG, "token %d has no block (table holds %zu)", token, t->ids.size());
    *block_id = t->ids[idx];
    *offset = token % bs;
    return GSP_OK;
}

int gsp_block_table_block_id(const gsp_block_table* t, int32_t index) {
    gsp::clear_error();
    if (!t || index < 0 || index >= (int32_t)t->ids.size()) {
        gsp::fail(GSP_E_INVALID_ARG, "block index %d out of range", index);
        return -1;
    }
    return t->ids[index];
}

int gsp_block_table_token_count(const gsp_block_table* t) { return t ? t->token_count : 0; }

int gsp_block_table_block_count(const gsp_block_table* t) { return t ? (int)t->ids.size() : 0; }

int gsp_block_table_ids(const gsp_block_table* t, int32_t* out, int32_t cap) {
    if (!t) return 0;
    const int32_t n = (int32_t)t->ids.size();
    if (out && cap > 0) std::copy(t->ids.begin(), t->ids.begin() + std::min(n, cap), out);
    return n;
}

void gsp_block_table_release_all(gsp_block_table* t) {
    if (!t) return;
    for (int32_t id : t->ids) t->alloc->release(id);
    t->ids.clear();
    t->token_count = 0;
}

}  // extern "C"
