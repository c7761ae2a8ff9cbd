// The block-id half of PagedBlockPool shared by the host metadata
// (gsp_host_meta.cpp, host code only: it builds without HIP) and the runtime,
// which attaches a device pool for copy-on-write page copies.
#pragma once

#include <atomic>
#include <cstdint>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/glacier_paged.h"

struct gsp_block_allocator {
    int32_t total = 0;
    int32_t block_size = 0;
    std::mutex stack_mu;
    std::vector<int32_t> free_stack;  // back() is the top of the LIFO stack
    std::unique_ptr<std::atomic<int32_t>[]> allocated;
    std::unique_ptr<std::atomic<int32_t>[]> refs;
    std::unique_ptr<std::atomic<uint64_t>[]> hashes;  // prefix hash bound to each block (0: none)
    std::mutex map_mu;
    std::unordered_map<uint64_t, int32_t> prefix_map;  // prefix hash -> block
    // Copy-on-write page copy of an attached device pool (gsp_pool_copy_block),
    // or null: a fork then only allocates, as the reference's metadata-only
    // pool does.
    gsp_ctx* ctx = nullptr;
    gsp_pool* pool = nullptr;
    int (*copy_page)(gsp_ctx*, gsp_pool*, int32_t src, int32_t dst, int32_t valid_tokens) = nullptr;

    bool try_allocate(int32_t* id) {
        int32_t b;
        {
            std::lock_guard<std::mutex> lk(stack_mu);
            if (free_stack.empty()) {
                *id = -1;
                return false;
            }
            b = free_stack.back();
            free_stack.pop_back();
        }
        allocated[b].store(1);
        refs[b].store(1);
        hashes[b].store(0);
        *id = b;
        return true;
    }

    int32_t release(int32_t id) {
        if (id < 0 || id >= total) return 0;
        const int32_t remaining = refs[id].fetch_sub(1) - 1;
        if (remaining < 0) {
            refs[id].store(0);
            return 0;
        }
        if (remaining == 0) {
            // A freed block leaves the prefix cache, unless its hash has since
            // been bound to another block (:263-271).
            const uint64_t h = hashes[id].load();
            if (h != 0) {
                {
                    std::lock_guard<std::mutex> lk(map_mu);
                    const auto it = prefix_map.find(h);
                    if (it != prefix_map.end() && it->second == id) prefix_map.erase(it);
                }
                hashes[id].store(0);
            }
            int32_t expected = 1;
            if (allocated[id].compare_exchange_strong(expected, 0)) {
                std::lock_guard<std::mutex> lk(stack_mu);
                free_stack.push_back(id);
            }
        }
        return remaining;
    }
};

struct gsp_block_table {
    gsp_block_allocator* alloc = nullptr;
    std::vector<int32_t> ids;
    int32_t token_count = 0;
};

