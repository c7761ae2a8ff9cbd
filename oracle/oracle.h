/*
 * CPU oracle for the paged-attention step — TEST INFRASTRUCTURE ONLY.
 *
 * A C++ restatement of the reference's CPU path, used by tests/ as the parity
 * checker and by bench.py's cpu_baseline leg as the timed CPU baseline.  No
 * product code links, loads or calls it.
 *
 * Restated from (reference paths relative to the Glacier.Serve tree):
 *   PagedAttentionKernel.ComputeAttention   PagedAttentionKernel.cs:17-372
 *   PagedBlockPool layout / Store           PagedBlockPool.cs:61-161
 *   PagedBlockPool free stack / refcounts   PagedBlockPool.cs:112-121,178-299,332-353
 *   BlockTable                              BlockTable.cs:13-117
 *   decode / prefill call order             PagedTransformerRunner.cs:521-656, 362-474
 *   RoPE before the store                   PagedTransformerRunner.cs:253-267, 436-449, 619-634
 *   YaRN / partial RoPE arguments           PagedTransformerRunner.cs:86-104, 253-264
 *
 * Parity status of each function is stated at its declaration.
 */
#ifndef GLACIER_ORACLE_H
#define GLACIER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Host pool: fp32 arenas in the reference layout
 * K[block][layer][hkv][slot][head_dim], V[block][layer][hkv][slot][v_head_dim]. */
typedef struct orc_pool {
    const float* k;
    const float* v;
    int32_t total_blocks;
    int32_t layers;
    int32_t heads_kv;
    int32_t head_dim;
    int32_t v_head_dim;
    int32_t block_size;
} orc_pool;

/* A BlockTable: its AsSpan() ids and TokenCount. */
typedef struct orc_table {
    const int32_t* ids;
    int32_t n_ids;
    int32_t token_count;
} orc_table;

enum { ORC_OK = 0, ORC_E_RANGE = 1, ORC_E_UNSUPPORTED = 2 };
enum { ORC_ISA_AUTO = -1, ORC_ISA_SCALAR = 0, ORC_ISA_AVX2 = 1, ORC_ISA_AVX512 = 2 };

/* Widest ISA this host supports (ORC_ISA_*), the analogue of
 * Vector512/Vector256.IsHardwareAccelerated. */
int orc_host_isa(void);

/* ComputeAttention (PagedAttentionKernel.cs:17-372).  Returns ORC_E_RANGE
 * where the reference throws ArgumentOutOfRangeException (:34-39) and when a
 * block index falls outside the table or pool (List indexer / pointer range);
 * ORC_E_UNSUPPORTED for a non-NULL sink (its Softmax semantics live in closed
 * code).  totalTokens == 0 returns ORC_OK with `out` untouched (:41-42).
 * n_threads plays Parallel.For over query heads (:48); isa picks the PV path
 * (:75-370).  head_scores: [n_heads][max_seq_len] scratch (:52).
 * Parity: QK dot order and softmax exp are restatements of closed
 * QuantKernels.VecDotF32/Softmax (unpinned beyond tolerance); every other
 * step follows the reference exactly. */
int orc_compute_attention(const orc_pool* pool, const orc_table* table, int32_t stage_layer,
                          int32_t model_layer, int32_t pos, const float* q, float* out,
                          int32_t n_heads, int32_t n_heads_kv, int32_t head_dim, int32_t v_head_dim,
                          float attn_scale, float* head_scores, int32_t max_seq_len,
                          const float* sink_logit, int32_t n_threads, int32_t isa);

/* Rotary position embedding as the reference applies it before the store
 * (PagedTransformerRunner.cs:253-267: QuantKernels.RoPE(q, k, nHeads, nHeadsKv,
 * headDim, pos, freqBase), then PagedBlockPool.Store).  Rotates n_vec vectors
 * of `dim` floats in place: pair j < dim/2 turns by
 * pos * freq_base^(-2j/dim), pairing (x[2j], x[2j+1]) for ORC_ROPE_PAIRS or
 * (x[j], x[j + dim/2]) for ORC_ROPE_HALVES; angles, sines and products in
 * fp64.  Parity: QuantKernels.RoPE is closed code; this is the textbook
 * definition (Su et al., RoFormer, 2021), and which pairing the reference
 * uses is unpinned. */
enum { ORC_ROPE_PAIRS = 0, ORC_ROPE_HALVES = 1 };
void orc_rope(float* x, int32_t n_vec, int32_t dim, int32_t pos, double freq_base, int32_t style);

/* The same rotation with the runner's optional arguments, QuantKernels.RoPE(...,
 * ropeFreqs, ropeDim, invFreqTable, mscale) (PagedTransformerRunner.cs:253-264,
 * 436-447, 619-631): only the first rope_dim dims of each vector are paired
 * (PAIRS: (x[2j], x[2j+1]); HALVES: (x[j], x[j + rope_dim/2])), the rest are
 * left as they are; pair j's angle is pos * inv_freq[j] (freq_base^(-2j/rope_dim)
 * when inv_freq is NULL), divided by freq_factors[j] when given; the rotated
 * pair is multiplied by mscale.  All in fp64.  Parity: the rotation of a
 * given table is pinned by closed forms (tests/test_rope.py); how the closed
 * QuantKernels.RoPE combines a table with ropeFreqs, and whether it scales
 * the dims past ropeDim, is unpinned (no reference test covers them). */
void orc_rope_ex(float* x, int32_t n_vec, int32_t dim, int32_t pos, double freq_base, int32_t style,
                 int32_t rope_dim, const float* inv_freq, const float* freq_factors, double mscale);

/* One engine step the way the reference runner drives the kernel: rows in
 * order (PagedTransformerRunner.cs:605-656), query token i of a row at
 * positions[b] + i (prefill, :454-474).  q is [total_q][n_heads][head_dim],
 * out is [total_q][n_heads][v_head_dim]; q_lens NULL means all 1.  Returns the
 * first failing status. */
int orc_attention_step(const orc_pool* pool, int32_t layer, int32_t num_rows,
                       const int32_t* positions, const int32_t* q_lens,
                       const int32_t* token_counts, const int32_t* bt_offsets,
                       const int32_t* bt_ids, const float* q, float* out, int32_t n_heads,
                       float attn_scale, int32_t max_seq_len, int32_t n_threads, int32_t isa);

/* Dense fp64 attention over the gathered K/V of one query token: the
 * textbook definition softmax(q.K^T * scale) V with double accumulation.
 * Same bounds rules as orc_compute_attention; out is written as fp64. */
int orc_attention_fp64(const orc_pool* pool, const orc_table* table, int32_t layer, int32_t pos,
                       const float* q, double* out, int32_t n_heads, double attn_scale,
                       int32_t max_seq_len);

/* Free stack / refcounts (PagedBlockPool.cs:112-121,178-299) and BlockTable
 * (BlockTable.cs:13-117), metadata only.  Pinned by the reference KATs. */
typedef struct orc_alloc orc_alloc;
typedef struct orc_btab orc_btab;

orc_alloc* orc_alloc_create(int32_t total_blocks, int32_t block_size);
void orc_alloc_destroy(orc_alloc* a);
int orc_alloc_try_allocate(orc_alloc* a, int32_t* id);
int orc_alloc_retain(orc_alloc* a, int32_t id); /* -1 where the reference throws */
int orc_alloc_release(orc_alloc* a, int32_t id);
int orc_alloc_ref_count(const orc_alloc* a, int32_t id);
int orc_alloc_free_count(const orc_alloc* a);
/* Prefix cache (PagedBlockPool.cs:194-234): find returns 1 and raises the
 * refcount when a live block holds the hash; bind returns -1 where the
 * reference throws (id outside the pool, hash 0). */
int orc_alloc_find_prefix(orc_alloc* a, uint64_t hash, int32_t* id);
int orc_alloc_bind_prefix(orc_alloc* a, uint64_t hash, int32_t id);

orc_btab* orc_btab_create(orc_alloc* a);
void orc_btab_destroy(orc_btab* t);
void orc_btab_attach_prefix(orc_btab* t, const int32_t* ids, int32_t n, int32_t token_count);
int orc_btab_append_token(orc_btab* t, int32_t* block_id, int32_t* offset);
int orc_btab_append_tokens(orc_btab* t, int32_t n); /* appended count */
int orc_btab_token_count(const orc_btab* t);
int orc_btab_ids(const orc_btab* t, int32_t* out, int32_t cap);
void orc_btab_release_all(orc_btab* t);

#ifdef __cplusplus
}
#endif

#endif
