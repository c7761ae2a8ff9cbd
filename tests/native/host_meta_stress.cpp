// Concurrency tests of the host block metadata (free stack, refcounts, prefix
// cache, BlockTable copy-on-write) through the C ABI, with real threads.  The
// reference's pool is used from several threads at once: HTTP admission looks
// up cached prefixes (ContinuousBatchEngine.cs:229-251) while the engine loop
// allocates and releases.  The cases port the reference's adversarial tests:
//   cow16   PrefixHashKvCacheAdversarialTests.cs:43-107  (16 concurrent COW forks)
//   aba     PrefixHashKvCacheAdversarialTests.cs:209-265 (recycled-block ABA race)
//   churn32 PrefixHashKvCacheAdversarialTests.cs:439-467 (32-thread prefix churn)
// plus `engine`, an engine thread growing and evicting tables while four
// admission threads look up prefixes.  Built plain, with ThreadSanitizer and
// with AddressSanitizer + UndefinedBehaviorSanitizer (tests/native/Makefile);
// each run exits non-zero on the first failed check.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

#include "glacier_paged.h"

namespace {

int g_failures = 0;

#define CHECK(cond)                                                                 \
    do {                                                                            \
        if (!(cond)) {                                                              \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            ++g_failures;                                                           \
            return;                                                                 \
        }                                                                           \
    } while (0)

template <typename F>
void run_threads(int n, F f) {
    std::vector<std::thread> ts;
    ts.reserve(n);
    for (int i = 0; i < n; ++i) ts.emplace_back(f, i);
    for (auto& t : ts) t.join();
}

void refcounts_non_negative(gsp_block_allocator* a) {
    for (int b = 0; b < gsp_block_allocator_total(a); ++b) CHECK(gsp_block_allocator_ref_count(a, b) >= 0);
}

// 16 sequences share one block holding 8 tokens; all append token 8 at once.
// Each must end on a private page at offset 8 (15 forks and the last holder
// keeps the original), and releasing them all returns every block.
void cow16() {
    const int n = 16;
    gsp_block_allocator* a = nullptr;
    CHECK(gsp_block_allocator_create(64, 16, &a) == GSP_OK);
    int32_t shared = -1;
    CHECK(gsp_block_allocator_try_allocate(a, &shared) == 1);
    for (int i = 1; i < n; ++i) CHECK(gsp_block_allocator_retain(a, shared) == i + 1);
    std::vector<gsp_block_table*> tables(n);
    for (int i = 0; i < n; ++i) {
        CHECK(gsp_block_table_create(a, &tables[i]) == GSP_OK);
        CHECK(gsp_block_table_attach_prefix(tables[i], &shared, 1, 8) == GSP_OK);
    }
    std::vector<int32_t> ids(n, -1), offs(n, -1);
    std::atomic<int> ready{0};
    run_threads(n, [&](int i) {
        // Start the appends together: each thread waits until all are running.
        ready.fetch_add(1);
        while (ready.load() < n) std::this_thread::yield();
        int32_t b, o;
        if (gsp_block_table_append_token(tables[i], &b, &o) == 1) {
            ids[i] = b;
            offs[i] = o;
        }
    });
    for (int i = 0; i < n; ++i) {
        CHECK(offs[i] == 8);
        CHECK(ids[i] == gsp_block_table_block_id(tables[i], 0));
        CHECK(gsp_block_allocator_ref_count(a, ids[i]) == 1);
        for (int j = 0; j < i; ++j) CHECK(ids[i] != ids[j]);
    }
    CHECK(gsp_block_allocator_free_count(a) == 64 - n);
    for (int i = 0; i < n; ++i) {
        gsp_block_table_release_all(tables[i]);
        gsp_block_table_destroy(tables[i]);
    }
    CHECK(gsp_block_allocator_free_count(a) == 64);
    refcounts_non_negative(a);
    gsp_block_allocator_destroy(a);
}

// Recycling threads bind a block to hash A, free it, reallocate it and bind
// hash B; lookup threads search hash A.  A hit must hold a live reference
// (refcount > 0) and still carry hash A.
void aba() {
    gsp_block_allocator* a = nullptr;
    CHECK(gsp_block_allocator_create(4, 16, &a) == GSP_OK);
    const uint64_t hash_a = 0xAAAAAAAAAAAAAAAAull, hash_b = 0xBBBBBBBBBBBBBBBBull;
    std::atomic<int> violations{0}, hits{0};
    run_threads(8, [&](int w) {
        for (int i = w; i < 10000; i += 8) {
            if ((i & 1) == 0) {
                int32_t b;
                if (gsp_block_allocator_try_allocate(a, &b) == 1) {
                    gsp_block_allocator_bind_prefix(a, hash_a, b);
                    std::this_thread::yield();
                    gsp_block_allocator_release(a, b);
                    int32_t r;
                    if (gsp_block_allocator_try_allocate(a, &r) == 1) {
                        gsp_block_allocator_bind_prefix(a, hash_b, r);
                        std::this_thread::yield();
                        gsp_block_allocator_release(a, r);
                    }
                }
            } else {
                int32_t f;
                if (gsp_block_allocator_find_prefix(a, hash_a, &f) == 1) {
                    hits.fetch_add(1);
                    if (gsp_block_allocator_ref_count(a, f) <= 0) violations.fetch_add(1);
                    gsp_block_allocator_release(a, f);
                }
            }
        }
    });
    CHECK(violations.load() == 0);
    refcounts_non_negative(a);
    CHECK(gsp_block_allocator_free_count(a) == 4);
    std::printf("aba: %d hits on hash A, 0 violations\n", hits.load());
    gsp_block_allocator_destroy(a);
}

// 32 threads allocate, bind one of 16 hashes, find it and release both
// references.  Everything converges back to a full free stack.
void churn32() {
    gsp_block_allocator* a = nullptr;
    CHECK(gsp_block_allocator_create(64, 16, &a) == GSP_OK);
    std::atomic<int> bad{0};
    run_threads(32, [&](int w) {
        for (int i = w; i < 10000; i += 32) {
            const uint64_t hash = 0xAA000000ull + (uint64_t)(i % 16);
            int32_t b;
            if (gsp_block_allocator_try_allocate(a, &b) == 1) {
                gsp_block_allocator_bind_prefix(a, hash, b);
                int32_t f;
                if (gsp_block_allocator_find_prefix(a, hash, &f) == 1) {
                    if (f < 0 || f >= 64) bad.fetch_add(1);
                    gsp_block_allocator_release(a, f);
                }
                gsp_block_allocator_release(a, b);
            }
        }
    });
    CHECK(bad.load() == 0);
    refcounts_non_negative(a);
    CHECK(gsp_block_allocator_free_count(a) == 64);
    gsp_block_allocator_destroy(a);
}

// An engine thread admits sequences (appending tokens, binding full pages to
// their prefix hashes) and evicts them, while admission threads look the
// hashes up and attach hits to tables of their own, which they then grow
// onto fresh pages and release.  Afterwards every block is free again.
void engine() {
    const int total = 256;
    gsp_block_allocator* a = nullptr;
    CHECK(gsp_block_allocator_create(total, 16, &a) == GSP_OK);
    std::atomic<int> stop{0}, bad{0};
    std::thread eng([&] {
        std::vector<gsp_block_table*> live;
        uint64_t seed = 12345;
        auto rnd = [&] {
            seed = seed * 6364136223846793005ull + 1442695040888963407ull;
            return (uint32_t)(seed >> 33);
        };
        for (int step = 0; step < 4000; ++step) {
            if (!live.empty() && rnd() % 100 < 45) {
                const size_t k = rnd() % live.size();
                gsp_block_table_release_all(live[k]);
                gsp_block_table_destroy(live[k]);
                live[k] = live.back();
                live.pop_back();
                continue;
            }
            gsp_block_table* t = nullptr;
            if (gsp_block_table_create(a, &t) != GSP_OK) {
                bad.fetch_add(1);
                break;
            }
            const int n = 1 + (int)(rnd() % 70);
            const int got = gsp_block_table_append_tokens(t, n);
            if (got < n) {
                gsp_block_table_release_all(t);
                gsp_block_table_destroy(t);
                continue;
            }
            // Full pages are bound to hash (prefix id, page index).
            for (int p = 0; p < n / 16; ++p)
                gsp_block_allocator_bind_prefix(a, 0x5000ull + (uint64_t)(n % 8) * 64 + p,
                                                gsp_block_table_block_id(t, p));
            live.push_back(t);
        }
        for (auto* t : live) {
            gsp_block_table_release_all(t);
            gsp_block_table_destroy(t);
        }
        stop.store(1);
    });
    run_threads(4, [&](int w) {
        uint64_t k = (uint64_t)w;
        while (!stop.load()) {
            k = k * 2862933555777941757ull + 3037000493ull;
            const uint64_t hash = 0x5000ull + ((k >> 20) % 8) * 64 + ((k >> 40) % 4);
            int32_t f;
            if (gsp_block_allocator_find_prefix(a, hash, &f) != 1) continue;
            if (gsp_block_allocator_ref_count(a, f) <= 0) bad.fetch_add(1);
            gsp_block_table* t = nullptr;
            if (gsp_block_table_create(a, &t) != GSP_OK) {
                gsp_block_allocator_release(a, f);
                bad.fetch_add(1);
                continue;
            }
            gsp_block_table_attach_prefix(t, &f, 1, 16);  // the attached page keeps the lookup's reference
            gsp_block_table_append_tokens(t, 3);          // allocates a fresh page (16 is a page boundary)
            gsp_block_table_release_all(t);
            gsp_block_table_destroy(t);
        }
    });
    eng.join();
    CHECK(bad.load() == 0);
    refcounts_non_negative(a);
    CHECK(gsp_block_allocator_free_count(a) == total);
    gsp_block_allocator_destroy(a);
}

}  // namespace

int main() {
    cow16();
    aba();
    churn32();
    engine();
    if (g_failures) {
        std::fprintf(stderr, "%d check(s) failed\n", g_failures);
        return 1;
    }
    std::printf("host metadata concurrency: all cases passed\n");
    return 0;
}
