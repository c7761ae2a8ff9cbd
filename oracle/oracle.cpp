// CPU oracle for the paged-attention step — TEST INFRASTRUCTURE ONLY.
// Used by tests/ as the parity checker and timed by bench.py's cpu_baseline
// leg; the product library never links or loads it.  See oracle.h for the
// reference file:line each function restates.
#include "oracle.h"

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <vector>

namespace {

struct Geometry {
    int64_t head_k, layer_k, block_k;
    int64_t head_v, layer_v, block_v;
};

// PagedBlockPool strides (PagedBlockPool.cs:77-83).
Geometry strides(const orc_pool* p) {
    Geometry g;
    g.head_k = (int64_t)p->block_size * p->head_dim;
    g.layer_k = (int64_t)p->heads_kv * g.head_k;
    g.block_k = (int64_t)p->layers * g.layer_k;
    g.head_v = (int64_t)p->block_size * p->v_head_dim;
    g.layer_v = (int64_t)p->heads_kv * g.head_v;
    g.block_v = (int64_t)p->layers * g.layer_v;
    return g;
}

// GetKeyPtr / GetValuePtr (PagedBlockPool.cs:124-145).
inline const float* key_ptr(const orc_pool* p, const Geometry& g, int b, int l, int h, int t) {
    return p->k + (int64_t)b * g.block_k + (int64_t)l * g.layer_k + (int64_t)h * g.head_k + (int64_t)t * p->head_dim;
}
inline const float* value_ptr(const orc_pool* p, const Geometry& g, int b, int l, int h, int t) {
    return p->v + (int64_t)b * g.block_v + (int64_t)l * g.layer_v + (int64_t)h * g.head_v + (int64_t)t * p->v_head_dim;
}

bool cpu_has_avx512() { return __builtin_cpu_supports("avx512f"); }
bool cpu_has_avx2() { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }

// ---- VecDotF32 restatement (external QuantKernels, PagedAttentionKernel.cs:64).
float dot_scalar(const float* a, const float* b, int n) {
    float acc = 0.f;
    for (int i = 0; i < n; ++i) acc = std::fma(a[i], b[i], acc);
    return acc;
}

__attribute__((target("avx2,fma"))) float dot_avx2(const float* a, const float* b, int n) {
    __m256 acc = _mm256_setzero_ps();
    int i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    float r = _mm_cvtss_f32(s);
    for (; i < n; ++i) r = std::fma(a[i], b[i], r);
    return r;
}

__attribute__((target("avx512f"))) float dot_avx512(const float* a, const float* b, int n) {
    __m512 acc = _mm512_setzero_ps();
    int i = 0;
    for (; i + 16 <= n; i += 16) acc = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), acc);
    float r = _mm512_reduce_add_ps(acc);
    for (; i < n; ++i) r = std::fma(a[i], b[i], r);
    return r;
}

// ---- Softmax restatement (external QuantKernels, PagedAttentionKernel.cs:70).
void softmax(float* s, int n) {
    float mx = s[0];
    for (int i = 1; i < n; ++i) mx = std::max(mx, s[i]);
    float sum = 0.f;
    for (int i = 0; i < n; ++i) {
        s[i] = std::exp(s[i] - mx);
        sum += s[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; ++i) s[i] *= inv;
}

struct HeadJob {
    const orc_pool* pool;
    Geometry g;
    const orc_table* table;
    int layer, total, block_count, head_dim, v_head_dim, group;
    float scale;
    const float* q;
    float* out;
    float* scores;
    int max_seq_len;
};

// PV accumulation with `NACC` register accumulators of `W`-float vectors
// (PagedAttentionKernel.cs:75-325): acc_j = fma(w, v[j*W..], acc_j) in token
// order, stored at the end.
template <int NACC>
__attribute__((target("avx512f"))) void pv_avx512(const HeadJob& J, int hkv, const float* sc, float* oh) {
    __m512 acc[NACC];
    for (int j = 0; j < NACC; ++j) acc[j] = _mm512_setzero_ps();
    const int bs = J.pool->block_size;
    for (int b = 0; b < J.block_count; ++b) {
        const int pb = J.table->ids[b];
        const int base = b * bs;
        const int tib = std::min(bs, J.total - base);
        for (int t = 0; t < tib; ++t) {
            const __m512 w = _mm512_set1_ps(sc[base + t]);
            const float* vp = value_ptr(J.pool, J.g, pb, J.layer, hkv, t);
            for (int j = 0; j < NACC; ++j) acc[j] = _mm512_fmadd_ps(w, _mm512_loadu_ps(vp + 16 * j), acc[j]);
        }
    }
    for (int j = 0; j < NACC; ++j) _mm512_storeu_ps(oh + 16 * j, acc[j]);
}

template <int NACC>
__attribute__((target("avx2,fma"))) void pv_avx2(const HeadJob& J, int hkv, const float* sc, float* oh) {
    __m256 acc[NACC];
    for (int j = 0; j < NACC; ++j) acc[j] = _mm256_setzero_ps();
    const int bs = J.pool->block_size;
    for (int b = 0; b < J.block_count; ++b) {
        const int pb = J.table->ids[b];
        const int base = b * bs;
        const int tib = std::min(bs, J.total - base);
        for (int t = 0; t < tib; ++t) {
            const __m256 w = _mm256_set1_ps(sc[base + t]);
            const float* vp = value_ptr(J.pool, J.g, pb, J.layer, hkv, t);
            for (int j = 0; j < NACC; ++j) acc[j] = _mm256_fmadd_ps(w, _mm256_loadu_ps(vp + 8 * j), acc[j]);
        }
    }
    for (int j = 0; j < NACC; ++j) _mm256_storeu_ps(oh + 8 * j, acc[j]);
}

// Generic path (PagedAttentionKernel.cs:326-370): zero, then per token a
// 16-wide, an 8-wide and a scalar (unfused) sweep.
__attribute__((target("avx512f"))) void pv_generic_512(float* oh, const float* vp, float w, int dv, int* d) {
    const __m512 vw = _mm512_set1_ps(w);
    for (; *d <= dv - 16; *d += 16)
        _mm512_storeu_ps(oh + *d, _mm512_fmadd_ps(vw, _mm512_loadu_ps(vp + *d), _mm512_loadu_ps(oh + *d)));
}
__attribute__((target("avx2,fma"))) void pv_generic_256(float* oh, const float* vp, float w, int dv, int* d) {
    const __m256 vw = _mm256_set1_ps(w);
    for (; *d <= dv - 8; *d += 8)
        _mm256_storeu_ps(oh + *d, _mm256_fmadd_ps(vw, _mm256_loadu_ps(vp + *d), _mm256_loadu_ps(oh + *d)));
}

void pv_generic(const HeadJob& J, int hkv, const float* sc, float* oh, int isa) {
    const int dv = J.v_head_dim;
    for (int d = 0; d < dv; ++d) oh[d] = 0.f;
    const int bs = J.pool->block_size;
    for (int b = 0; b < J.block_count; ++b) {
        const int pb = J.table->ids[b];
        const int base = b * bs;
        const int tib = std::min(bs, J.total - base);
        for (int t = 0; t < tib; ++t) {
            const float w = sc[base + t];
            const float* vp = value_ptr(J.pool, J.g, pb, J.layer, hkv, t);
            int d = 0;
            if (isa >= ORC_ISA_AVX512 && dv >= 16) pv_generic_512(oh, vp, w, dv, &d);
            if (isa >= ORC_ISA_AVX2 && dv - d >= 8) pv_generic_256(oh, vp, w, dv, &d);
            for (; d < dv; ++d) oh[d] += w * vp[d];
        }
    }
}

void run_head(const HeadJob& J, int h, int isa) {
    const int hkv = h / J.group;                             // :50
    const float* qh = J.q + (int64_t)h * J.head_dim;         // :51
    float* sc = J.scores + (int64_t)h * J.max_seq_len;       // :52
    const int bs = J.pool->block_size;
    // 1. QK^T page by page (:55-67): the scale multiplies the finished dot.
    for (int b = 0; b < J.block_count; ++b) {
        const int pb = J.table->ids[b];
        const int base = b * bs;
        const int tib = std::min(bs, J.total - base);
        for (int t = 0; t < tib; ++t) {
            const float* kp = key_ptr(J.pool, J.g, pb, J.layer, hkv, t);
            float dot;
            if (isa >= ORC_ISA_AVX512) dot = dot_avx512(qh, kp, J.head_dim);
            else if (isa >= ORC_ISA_AVX2) dot = dot_avx2(qh, kp, J.head_dim);
            else dot = dot_scalar(qh, kp, J.head_dim);
            sc[base + t] = dot * J.scale;
        }
    }
    // 2. Softmax over the valid tokens (:70).
    softmax(sc, J.total);
    // 3. PV (:73-370), dispatched as the reference does.
    float* oh = J.out + (int64_t)h * J.v_head_dim;
    const int dv = J.v_head_dim;
    if (isa >= ORC_ISA_AVX512 && dv == 128) pv_avx512<8>(J, hkv, sc, oh);
    else if (isa >= ORC_ISA_AVX512 && dv == 64) pv_avx512<4>(J, hkv, sc, oh);
    else if (isa >= ORC_ISA_AVX512 && dv == 256) pv_avx512<16>(J, hkv, sc, oh);
    else if (isa >= ORC_ISA_AVX2 && dv == 64) pv_avx2<8>(J, hkv, sc, oh);
    else if (isa >= ORC_ISA_AVX2 && dv == 128) pv_avx2<16>(J, hkv, sc, oh);
    else pv_generic(J, hkv, sc, oh, isa);
}

int resolve_isa(int isa) {
    const int host = orc_host_isa();
    if (isa < 0 || isa > host) return host;
    return isa;
}

// Bounds and geometry checks shared by the fp32 and fp64 paths.
int check_call(const orc_pool* pool, const orc_table* table, int layer, int pos, int n_heads, int n_heads_kv,
               int head_dim, int v_head_dim, int max_seq_len, int* total_out, int* block_count_out) {
    if (!pool || !table) return ORC_E_RANGE;
    if (max_seq_len <= 0) return ORC_E_RANGE;                          // :34-35
    if (pos < 0 || pos >= max_seq_len) return ORC_E_RANGE;             // :36-37
    if (table->token_count > max_seq_len) return ORC_E_RANGE;          // :38-39
    const int total = std::min(table->token_count, pos + 1);           // :41
    *total_out = total;
    *block_count_out = 0;
    if (total <= 0) return ORC_OK;                                     // :42
    if (n_heads_kv <= 0 || n_heads <= 0 || n_heads < n_heads_kv) return ORC_E_RANGE;
    const int group = n_heads / n_heads_kv;
    if ((n_heads - 1) / group >= pool->heads_kv) return ORC_E_RANGE;   // pointer would leave the pool
    if (head_dim != pool->head_dim || v_head_dim != pool->v_head_dim) return ORC_E_RANGE;
    if (layer < 0 || layer >= pool->layers) return ORC_E_RANGE;
    const int bs = pool->block_size;
    const int block_count = (total + bs - 1) / bs;                     // :46
    if (block_count > table->n_ids) return ORC_E_RANGE;                // GetBlockId indexer
    for (int b = 0; b < block_count; ++b)
        if (table->ids[b] < 0 || table->ids[b] >= pool->total_blocks) return ORC_E_RANGE;
    *block_count_out = block_count;
    return ORC_OK;
}

}  // namespace

extern "C" {

int orc_host_isa(void) {
    if (cpu_has_avx512()) return ORC_ISA_AVX512;
    if (cpu_has_avx2()) return ORC_ISA_AVX2;
    return ORC_ISA_SCALAR;
}

int orc_compute_attention(const orc_pool* pool, const orc_table* table, int32_t stage_layer, int32_t model_layer,
                          int32_t pos, const float* q, float* out, int32_t n_heads, int32_t n_heads_kv,
                          int32_t head_dim, int32_t v_head_dim, float attn_scale, float* head_scores,
                          int32_t max_seq_len, const float* sink_logit, int32_t n_threads, int32_t isa) {
    (void)model_layer;  // unused by the reference (PagedAttentionKernel.cs:19)
    int total = 0, block_count = 0;
    int rc = check_call(pool, table, stage_layer, pos, n_heads, n_heads_kv, head_dim, v_head_dim, max_seq_len,
                        &total, &block_count);
    if (rc != ORC_OK || total <= 0) return rc;
    if (sink_logit) return ORC_E_UNSUPPORTED;
    std::vector<float> own;
    if (!head_scores) {
        own.resize((size_t)n_heads * max_seq_len);
        head_scores = own.data();
    }
    HeadJob J;
    J.pool = pool;
    J.g = strides(pool);
    J.table = table;
    J.layer = stage_layer;
    J.total = total;
    J.block_count = block_count;
    J.head_dim = head_dim;
    J.v_head_dim = v_head_dim;
    J.group = n_heads / n_heads_kv;  // :44
    J.scale = attn_scale;
    J.q = q;
    J.out = out;
    J.scores = head_scores;
    J.max_seq_len = max_seq_len;
    const int use = resolve_isa(isa);
    const int nt = std::max(1, n_threads);
    // Parallel.For(0, nHeads, ...) (:48).
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt) if (nt > 1)
    for (int h = 0; h < n_heads; ++h) run_head(J, h, use);
    return ORC_OK;
}

int orc_attention_step(const orc_pool* pool, int32_t layer, int32_t num_rows, const int32_t* positions,
                       const int32_t* q_lens, const int32_t* token_counts, const int32_t* bt_offsets,
                       const int32_t* bt_ids, const float* q, float* out, int32_t n_heads, float attn_scale,
                       int32_t max_seq_len, int32_t n_threads, int32_t isa) {
    if (!pool) return ORC_E_RANGE;
    std::vector<float> scores((size_t)n_heads * std::max(1, max_seq_len));
    int64_t qi = 0;
    for (int b = 0; b < num_rows; ++b) {
        const int ql = q_lens ? q_lens[b] : 1;
        orc_table t;
        t.ids = bt_ids + bt_offsets[b];
        t.n_ids = bt_offsets[b + 1] - bt_offsets[b];
        t.token_count = token_counts[b];
        for (int i = 0; i < ql; ++i, ++qi) {
            int rc = orc_compute_attention(pool, &t, layer, layer, positions[b] + i,
                                           q + qi * (int64_t)n_heads * pool->head_dim,
                                           out + qi * (int64_t)n_heads * pool->v_head_dim, n_heads, pool->heads_kv,
                                           pool->head_dim, pool->v_head_dim, attn_scale, scores.data(), max_seq_len,
                                           nullptr, n_threads, isa);
            if (rc != ORC_OK) return rc;
        }
    }
    return ORC_OK;
}

int orc_attention_fp64(const orc_pool* pool, const orc_table* table, int32_t layer, int32_t pos, const float* q,
                       double* out, int32_t n_heads, double attn_scale, int32_t max_seq_len) {
    int total = 0, block_count = 0;
    int rc = check_call(pool, table, layer, pos, n_heads, pool ? pool->heads_kv : 0, pool ? pool->head_dim : 0,
                        pool ? pool->v_head_dim : 0, max_seq_len, &total, &block_count);
    if (rc != ORC_OK || total <= 0) return rc;
    const Geometry g = strides(pool);
    const int d = pool->head_dim, dv = pool->v_head_dim, bs = pool->block_size;
    const int group = n_heads / pool->heads_kv;
    std::vector<double> s(total);
    for (int h = 0; h < n_heads; ++h) {
        const int hkv = h / group;
        double mx = -INFINITY;
        for (int t = 0; t < total; ++t) {
            const float* kp = key_ptr(pool, g, table->ids[t / bs], layer, hkv, t % bs);
            double acc = 0.0;
            for (int e = 0; e < d; ++e) acc += (double)q[(int64_t)h * d + e] * (double)kp[e];
            s[t] = acc * attn_scale;
            mx = std::max(mx, s[t]);
        }
        double sum = 0.0;
        for (int t = 0; t < total; ++t) {
            s[t] = std::exp(s[t] - mx);
            sum += s[t];
        }
        for (int e = 0; e < dv; ++e) out[(int64_t)h * dv + e] = 0.0;
        for (int t = 0; t < total; ++t) {
            const float* vp = value_ptr(pool, g, table->ids[t / bs], layer, hkv, t % bs);
            const double w = s[t] / sum;
            for (int e = 0; e < dv; ++e) out[(int64_t)h * dv + e] += w * (double)vp[e];
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------ metadata */

struct orc_alloc {
    int32_t total, block_size;
    std::vector<int32_t> stack;  // back() = top
    std::vector<int32_t> allocated, refs;
    std::vector<uint64_t> hashes;              // _blockPrefixHashes
    std::map<uint64_t, int32_t> prefix_map;    // _prefixHashMap
};

struct orc_btab {
    orc_alloc* a;
    std::vector<int32_t> ids;
    int32_t token_count;
};

orc_alloc* orc_alloc_create(int32_t total_blocks, int32_t block_size) {
    if (total_blocks < 1 || block_size < 1) return nullptr;
    orc_alloc* a = new orc_alloc();
    a->total = total_blocks;
    a->block_size = block_size;
    a->allocated.assign(total_blocks, 0);
    a->refs.assign(total_blocks, 0);
    a->hashes.assign(total_blocks, 0);
    for (int32_t i = total_blocks - 1; i >= 0; --i) a->stack.push_back(i);  // :116-120
    return a;
}

void orc_alloc_destroy(orc_alloc* a) { delete a; }

int orc_alloc_try_allocate(orc_alloc* a, int32_t* id) {  // :178-189
    if (a->stack.empty()) {
        *id = -1;
        return 0;
    }
    *id = a->stack.back();
    a->stack.pop_back();
    a->allocated[*id] = 1;
    a->refs[*id] = 1;
    a->hashes[*id] = 0;
    return 1;
}

int orc_alloc_retain(orc_alloc* a, int32_t id) {  // :240-245
    if (id < 0 || id >= a->total) return -1;
    return ++a->refs[id];
}

int orc_alloc_release(orc_alloc* a, int32_t id) {  // :251-279
    if (id < 0 || id >= a->total) return 0;
    const int remaining = --a->refs[id];
    if (remaining < 0) {
        a->refs[id] = 0;
        return 0;
    }
    if (remaining == 0) {
        const uint64_t h = a->hashes[id];  // :265-270: drop the map entry only if it is still this block's
        if (h != 0) {
            const auto it = a->prefix_map.find(h);
            if (it != a->prefix_map.end() && it->second == id) a->prefix_map.erase(it);
            a->hashes[id] = 0;
        }
        if (a->allocated[id] == 1) {  // :272-275
            a->allocated[id] = 0;
            a->stack.push_back(id);
        }
    }
    return remaining;
}

int orc_alloc_find_prefix(orc_alloc* a, uint64_t hash, int32_t* id) {  // :194-220
    *id = -1;
    if (hash == 0) return 0;
    const auto it = a->prefix_map.find(hash);
    if (it == a->prefix_map.end()) return 0;
    const int32_t b = it->second;
    if (a->refs[b] <= 0) return 0;
    ++a->refs[b];
    if (a->hashes[b] != hash) {
        orc_alloc_release(a, b);
        return 0;
    }
    *id = b;
    return 1;
}

int orc_alloc_bind_prefix(orc_alloc* a, uint64_t hash, int32_t id) {  // :225-234; -1 where the reference throws
    if (id < 0 || id >= a->total || hash == 0) return -1;
    a->hashes[id] = hash;
    a->prefix_map[hash] = id;
    return 0;
}

int orc_alloc_ref_count(const orc_alloc* a, int32_t id) {
    if (id < 0 || id >= a->total) return 0;
    return a->refs[id];
}

int orc_alloc_free_count(const orc_alloc* a) { return (int)a->stack.size(); }

orc_btab* orc_btab_create(orc_alloc* a) {
    orc_btab* t = new orc_btab();
    t->a = a;
    t->token_count = 0;
    return t;
}

void orc_btab_destroy(orc_btab* t) { delete t; }

void orc_btab_attach_prefix(orc_btab* t, const int32_t* ids, int32_t n, int32_t token_count) {  // BlockTable.cs:31-39
    t->ids.insert(t->ids.end(), ids, ids + n);
    t->token_count = token_count;
}

int orc_btab_append_token(orc_btab* t, int32_t* block_id, int32_t* offset) {  // BlockTable.cs:46-80
    const int bs = t->a->block_size;
    if (t->token_count % bs == 0) {
        int32_t nb;
        if (!orc_alloc_try_allocate(t->a, &nb)) {
            *block_id = -1;
            *offset = -1;
            return 0;
        }
        t->ids.push_back(nb);
    } else {
        const int32_t last = t->ids.back();
        if (orc_alloc_ref_count(t->a, last) > 1) {
            int32_t forked;
            if (!orc_alloc_try_allocate(t->a, &forked)) {
                *block_id = -1;
                *offset = -1;
                return 0;
            }
            orc_alloc_release(t->a, last);
            t->ids.back() = forked;
        }
    }
    *block_id = t->ids.back();
    *offset = t->token_count % bs;
    t->token_count++;
    return 1;
}

int orc_btab_append_tokens(orc_btab* t, int32_t n) {
    int32_t b, o, done = 0;
    while (done < n && orc_btab_append_token(t, &b, &o)) ++done;
    return done;
}

int orc_btab_token_count(const orc_btab* t) { return t->token_count; }

int orc_btab_ids(const orc_btab* t, int32_t* out, int32_t cap) {
    const int n = (int)t->ids.size();
    if (out) std::copy(t->ids.begin(), t->ids.begin() + std::min(n, cap), out);
    return n;
}

void orc_btab_release_all(orc_btab* t) {  // BlockTable.cs:108-116
    for (int32_t id : t->ids) orc_alloc_release(t->a, id);
    t->ids.clear();
    t->token_count = 0;
}

}  // extern "C"

/* ------------------------------------------------------------------ RoPE */

extern "C" void orc_rope_ex(float* x, int32_t n_vec, int32_t dim, int32_t pos, double freq_base, int32_t style,
                            int32_t rope_dim, const float* inv_freq, const float* freq_factors, double mscale) {
    const int32_t half = rope_dim / 2;
    for (int32_t j = 0; j < half; ++j) {
        double rate = inv_freq ? (double)inv_freq[j] : std::pow(freq_base, -2.0 * j / rope_dim);
        if (freq_factors) rate /= (double)freq_factors[j];
        const double ang = (double)pos * rate;
        const double c = std::cos(ang) * mscale, s = std::sin(ang) * mscale;
        for (int32_t v = 0; v < n_vec; ++v) {
            float* p = x + (size_t)v * dim;
            float* a = style == ORC_ROPE_PAIRS ? p + 2 * j : p + j;
            float* b = style == ORC_ROPE_PAIRS ? p + 2 * j + 1 : p + j + half;
            const double x0 = *a, x1 = *b;
            *a = (float)(x0 * c - x1 * s);
            *b = (float)(x0 * s + x1 * c);
        }
    }
}

extern "C" void orc_rope(float* x, int32_t n_vec, int32_t dim, int32_t pos, double freq_base, int32_t style) {
    orc_rope_ex(x, n_vec, dim, pos, freq_base, style, dim, nullptr, nullptr, 1.0);
}
