/*
 * glacier_paged.h — C ABI of the MI355X (gfx950) ragged continuous-batch
 * paged-attention step.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, never
 * throws, and reports failure through a status code plus a thread-local
 * message (gsp_last_error).  Status codes map onto the reference's failure
 * behaviour:
 *   GSP_E_INVALID_ARG  <-> ArgumentOutOfRangeException / ArgumentNullException
 *                          (PagedAttentionKernel.cs:34-39, PagedBlockPool.cs:63-67,
 *                           PagedTransformerRunner.cs:533-540)
 *   GSP_E_OOM          <-> TryAllocateBlock == false / TryCreate == false
 *                          (PagedBlockPool.cs:178-189, CudaPagedTransformerRunner.cs:126-132)
 *   GSP_E_UNSUPPORTED  <-> IsModelSupportedOnGpu == false
 *                          (CudaPagedTransformerRunner.cs:381-460)
 *   GSP_E_HIP          <-> driver failure (CuDriver.Check)
 *
 * Threading: one gsp_ctx is driven by one thread at a time, as the reference
 * engine drives its runner from a single loop thread
 * (ContinuousBatchEngine.cs:333).  Distinct contexts are independent.  All
 * device work of a context is enqueued on one HIP stream; calls return after
 * enqueueing and gsp_sync() gives the reference's synchronous semantics.
 *
 * Ownership: the caller owns every host pointer for the duration of a call
 * only (the library copies what it keeps into its own pinned staging); the
 * library owns every allocation behind an opaque handle.  q/out/k/v device
 * pointers passed to compute calls are caller-owned device memory.
 */
#ifndef GLACIER_PAGED_H
#define GLACIER_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define GSP_ABI_VERSION 9
#define GSP_BLOCK_SIZE 16 /* PagedBlockPool.DefaultBlockSize (PagedBlockPool.cs:18) */
#define GSP_MAX_BLOCK_SIZE 4096 /* largest page size of a device pool */

typedef enum gsp_status {
    GSP_OK = 0,
    GSP_E_INVALID_ARG = 1,
    GSP_E_OOM = 2,
    GSP_E_UNSUPPORTED = 3,
    GSP_E_HIP = 4,
    GSP_E_STATE = 5 /* call order violated, e.g. attention before a step was packed */
} gsp_status;

typedef enum gsp_kv_dtype {
    GSP_KV_F32 = 0, /* host pool precision (PagedBlockPool.cs:36-37) */
    GSP_KV_F16 = 1  /* device pool precision of the reference GPU runner
                       (CudaPagedTransformerRunner.cs:118-119, KvCachePrecision.Fp16) */
} gsp_kv_dtype;

typedef struct gsp_ctx gsp_ctx;
typedef struct gsp_pool gsp_pool;
typedef struct gsp_block_allocator gsp_block_allocator;
typedef struct gsp_block_table gsp_block_table;

/* ------------------------------------------------------------------------ */
/* Diagnostics                                                              */
/* ------------------------------------------------------------------------ */

/* Message describing the last failing call on this thread ("" if none). */
const char* gsp_last_error(void);

int gsp_abi_version(void);

typedef struct gsp_device_info {
    char name[256];
    char arch[64];          /* e.g. "gfx950" */
    int32_t compute_units;
    int32_t wavefront_size;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width_bits;
    int64_t total_global_mem;
    int64_t lds_per_block;
} gsp_device_info;

/* Properties of HIP device `device`. */
int gsp_device_info_get(int device, gsp_device_info* out);

/* ------------------------------------------------------------------------ */
/* Context: GpuContext + TryCreate / Dispose                                 */
/* (CudaPagedTransformerRunner.cs:78-190, 490-523)                           */
/* ------------------------------------------------------------------------ */

/* Creates a context on HIP device `device` with its own stream.  Fails with
 * GSP_E_UNSUPPORTED when no gfx950 device is present (the caller then keeps
 * its CPU runner, as ContinuousBatchEngine.cs:139-168 does). */
int gsp_init(int device, gsp_ctx** out);
void gsp_shutdown(gsp_ctx* ctx);

/* Replaces the context's stream with a caller-owned hipStream_t (NULL restores
 * the context's own stream).  The caller keeps the stream alive. */
int gsp_set_stream(gsp_ctx* ctx, void* hip_stream);
void* gsp_get_stream(gsp_ctx* ctx);

/* Blocks until all work enqueued on the context's stream, and the upload of
 * the packed step, have finished.  After it the packed step may be read by a
 * graph capture (see gsp_attention_step). */
int gsp_sync(gsp_ctx* ctx);

/* ------------------------------------------------------------------------ */
/* Device KV pool: the device half of PagedBlockPool                         */
/* Layout (PagedBlockPool.cs:77-83,128-131,140-143), element offsets:        */
/*   K[block][layer][head_kv][slot < block_size][head_dim]                   */
/*   V[block][layer][head_kv][slot < block_size][v_head_dim]                 */
/* ------------------------------------------------------------------------ */

typedef struct gsp_pool_desc {
    int32_t total_blocks;
    int32_t layers;
    int32_t heads_kv;
    int32_t head_dim;
    int32_t v_head_dim;  /* <= 0 means head_dim (PagedBlockPool.cs:73) */
    int32_t block_size;  /* tokens per page, 1 .. GSP_MAX_BLOCK_SIZE (PagedBlockPool.cs:61-67
                            takes any blockSize >= 1) */
    int32_t kv_dtype;    /* gsp_kv_dtype */
} gsp_pool_desc;

/* Allocates zero-initialised K and V arenas in HBM
 * (CudaPagedTransformerRunner.cs:141-148).  GSP_E_OOM if they do not fit. */
int gsp_pool_create(gsp_ctx* ctx, const gsp_pool_desc* desc, gsp_pool** out);

/* Wraps caller-owned device arenas already laid out as above (the reference
 * hands raw dKPool/dVPool pointers to its kernels,
 * CudaPagedTransformerRunner.cs:352-360).  The library never frees them. */
int gsp_pool_wrap(gsp_ctx* ctx, const gsp_pool_desc* desc, void* k_dev, void* v_dev,
                  gsp_pool** out);
void gsp_pool_destroy(gsp_pool* pool);

/* Device addresses and byte sizes of the two arenas. */
int gsp_pool_arenas(const gsp_pool* pool, void** k_dev, void** v_dev, size_t* k_bytes,
                    size_t* v_bytes);

/* PagedBlockPool.Store (PagedBlockPool.cs:151-161), batched: token i of `n`
 * goes to slot slots[i] of block block_ids[i] in `layer`.  k_dev is
 * [n][heads_kv][head_dim] fp32, v_dev is [n][heads_kv][v_head_dim] fp32 (device
 * pointers); F16 pools round to nearest even on the device.  block_ids and
 * slots are host arrays. */
int gsp_pool_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n,
                          const int32_t* block_ids, const int32_t* slots, const float* k_dev,
                          const float* v_dev);

/* Pairings of gsp_rope_write_tokens. */
#define GSP_ROPE_PAIRS 0   /* pair j is (x[2j], x[2j+1]) */
#define GSP_ROPE_HALVES 1  /* pair j is (x[j], x[j + head_dim/2]) */

/* QuantKernels.RoPE(q, k, nHeads, nHeadsKv, headDim, pos, freqBase) followed
 * by PagedBlockPool.Store, fused and batched (PagedTransformerRunner.cs:253-267
 * and :620-634 for decode, :437-452 for a prefill chunk).  Token i sits at
 * position positions[i]; pair j of each of its heads turns by
 * positions[i] * freq_base^(-2j/head_dim).  q_dev ([n][n_heads][head_dim]
 * fp32, device) is rotated in place, or left alone with n_heads 0; k_dev is
 * rotated and stored, and v_dev stored as is, exactly where
 * gsp_pool_write_tokens stores them.  This is the domain of the reference's
 * GPU runner: RoPE over the full head, no frequency table, no YaRN
 * (CudaPagedTransformerRunner.cs:414-418; gsp_rope_write_tokens_ex below takes
 * the CPU runner's other arguments); head_dim even and at most 256.  The
 * reference's rotation lives in closed code, so `style` (GSP_ROPE_*) names the
 * pairing.  positions, block_ids and slots are host arrays. */
int gsp_rope_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n,
                          const int32_t* positions, const int32_t* block_ids,
                          const int32_t* slots, int32_t n_heads, float freq_base, int32_t style,
                          float* q_dev, const float* k_dev, const float* v_dev);

/* The K/V writes of a packed step, from the step's own device copy: no host
 * arrays, no upload and no host wait, so every layer of an engine tick reuses
 * the one upload of gsp_step_pack and the call can be captured.  Query token
 * i of row b (position positions[b] + i) stores k_dev[i] and v_dev[i]
 * ([total_q][heads_kv][head_dim] fp32, device) into the slot of that position
 * in the row's table, as the reference stores each new token before attending
 * (PagedTransformerRunner.cs:620-634 for decode, :437-452 for a prefill
 * chunk).  A token at a position >= the row's token_counts[b] has no slot and
 * is not stored.  gsp_rope_write_step first applies gsp_rope_write_tokens's
 * rotation at that position: q_dev ([total_q][n_heads][head_dim]) in place
 * (n_heads 0: left alone) and K on its way into the pool.  The pool must have
 * the geometry the step was packed for. */
int gsp_pool_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, const float* k_dev,
                        const float* v_dev);
int gsp_rope_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n_heads,
                        float freq_base, int32_t style, float* q_dev, const float* k_dev,
                        const float* v_dev);

/* The rotation with the optional arguments of the reference's CPU runner,
 * QuantKernels.RoPE(..., ropeFreqs, ropeDim, invFreqTable, mscale)
 * (PagedTransformerRunner.cs:253-264, :436-447 and :619-631; the YaRN table
 * and mscale are made at :86-104).  A zeroed struct with freq_base and style
 * set is gsp_rope_write_tokens's rotation.
 *   rope_dim      dims rotated per head, even, 2 <= rope_dim <= head_dim (0:
 *                 head_dim).  Pairs come from the first rope_dim dims (PAIRS:
 *                 (x[2j], x[2j+1]); HALVES: (x[j], x[j + rope_dim/2])); dims
 *                 from rope_dim on pass through, into the pool for K.
 *   inv_freq      NULL, or rope_dim/2 floats (host): pair j turns by
 *                 pos * inv_freq[j] (a YaRN table).  NULL: by
 *                 pos * freq_base^(-2j/rope_dim).
 *   freq_factors  NULL, or rope_dim/2 floats > 0 (host, the GGUF rope_freqs
 *                 tensor): pair j's angle is divided by freq_factors[j].
 *   mscale        the rotated pairs are scaled by it (YaRN's attention factor,
 *                 applied to Q and K alike); 0 means 1.
 * The angle rates (inv_freq / freq_factors, fp64) of the last table are kept
 * on the device; a call with another table first copies it there on the
 * context's stream, which a stream that is capturing into a graph refuses
 * with GSP_E_STATE (make one eager call with the table before capturing). */
typedef struct gsp_rope_spec {
  float freq_base;
  int32_t style;
  int32_t rope_dim;
  float mscale;
  const float* inv_freq;
  const float* freq_factors;
} gsp_rope_spec;

/* gsp_rope_write_tokens and gsp_rope_write_step with the rotation `rope`. */
int gsp_rope_write_tokens_ex(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n,
                             const int32_t* positions, const int32_t* block_ids,
                             const int32_t* slots, int32_t n_heads, const gsp_rope_spec* rope,
                             float* q_dev, const float* k_dev, const float* v_dev);
int gsp_rope_write_step_ex(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n_heads,
                           const gsp_rope_spec* rope, float* q_dev, const float* k_dev,
                           const float* v_dev);

/* Weight types of gsp_matmul_batch: the GGUF tensor type ids. */
#define GSP_WTYPE_F32 0
#define GSP_WTYPE_Q8_0 8
#define GSP_WTYPE_Q4_K 12
#define GSP_WTYPE_Q6_K 14

/* QuantKernels.MatMulBatch(type, weight, x, y, inDim, outDim, batchSize, xBlockSums)
 * (PagedTransformerRunner.cs:601-603 for Q/K/V, :659 for the attention
 * output): y[b][o] = sum_i W[o][i] * x[b][i] for b < batch, o < out_dim.  w_dev
 * holds out_dim rows of in_dim weights (the GGUF [in, out] layout), as fp32
 * (GSP_WTYPE_F32, 16-byte aligned), Q8_0 (GSP_WTYPE_Q8_0: per 32 weights a
 * little-endian fp16 scale d and 32 int8 q, w = d * q; 4-byte aligned), or
 * the K-quant super-blocks the reference GPU runner batches
 * (CudaPagedTransformerRunner.cs:470-473) in the public GGML layouts, 256
 * weights each: Q4_K (GSP_WTYPE_Q4_K, 144 bytes: fp16 d, fp16 dmin, 12 bytes
 * of 6-bit scales and mins, 128 bytes of 4-bit quants, w = d*sc*q - dmin*m;
 * 4-byte aligned) and Q6_K (GSP_WTYPE_Q6_K, 210 bytes: 128 bytes of low 4
 * bits, 64 of high 2 bits, 16 int8 scales, fp16 d, w = d*sc*(q - 32);
 * 2-byte aligned).  x_dev is [batch][in_dim] fp32 (16-byte aligned), y_dev
 * [batch][out_dim] fp32, overwritten; all device pointers.  Every weight is
 * decoded exactly (to the float32 value its format defines, or to its exact
 * fp16 quant and fp32 scale) and sums are fp32.  Q8_0, Q4_K and Q6_K
 * products with at least 16384 outputs (batch x out_dim) at up to 64 batch
 * rows, or at least 196608 outputs, take x as a scaled fp16 pair on the fp16
 * matrix cores (other products keep x in fp32, as F32 ones always do): each
 * element then carries an absolute error of at most
 * ~2^-22 of its row's largest |x| (~22 significant bits for elements near
 * the row max, fewer for much smaller ones; every finite x stays finite).
 * Results are the same bit for bit on every call.  in_dim must be a multiple
 * of 64 (256 for the K-quants; GSP_E_UNSUPPORTED otherwise, as for other
 * weight types); the reference's block sums are not needed by these types. */
int gsp_matmul_batch(gsp_ctx* ctx, int32_t w_type, const void* w_dev, const float* x_dev, float* y_dev,
                     int32_t in_dim, int32_t out_dim, int32_t batch);

/* PagedBlockPool.CopyBlockData (PagedBlockPool.cs:304-327): copies the first
 * min(valid_tokens, block_size) slots of every layer and KV head of block
 * `src` to block `dst`, on the device.  valid_tokens <= 0 is a no-op.  It only
 * enqueues a kernel, so copy-on-write forks of an attached pool may run on
 * several threads at once, as the reference's concurrent forks do. */
int gsp_pool_copy_block(gsp_ctx* ctx, gsp_pool* pool, int32_t src, int32_t dst,
                        int32_t valid_tokens);

/* Test/fixture support: synchronous byte copies between host memory and an
 * arena (which: 0 = K, 1 = V). */
int gsp_pool_upload(gsp_ctx* ctx, gsp_pool* pool, int32_t which, size_t offset_bytes,
                    const void* host, size_t bytes);
int gsp_pool_download(gsp_ctx* ctx, gsp_pool* pool, int32_t which, size_t offset_bytes,
                      void* host, size_t bytes);

/* ------------------------------------------------------------------------ */
/* Step packing: replaces the per-sequence UploadBlockTable copies           */
/* (CudaPagedTransformerRunner.cs:330-379) with one packed upload per step.  */
/* ------------------------------------------------------------------------ */

typedef struct gsp_step_desc {
    int32_t num_rows;            /* B: sequences in this engine step */
    int32_t max_seq_len;         /* maxSeqLen of the runner */
    const int32_t* positions;    /* [B] position of the row's first query token */
    const int32_t* q_lens;       /* [B] query tokens per row (NULL: all 1 = decode rows) */
    const int32_t* token_counts; /* [B] BlockTable.TokenCount after slot allocation */
    const int32_t* bt_offsets;   /* [B+1] CSR offsets into bt_ids */
    const int32_t* bt_ids;       /* concatenated BlockTable.AsSpan() of each row */
    int32_t n_bt_ids;            /* entries readable at bt_ids: the CSR must keep
                                    0 <= bt_offsets[b] <= bt_offsets[b+1] <= n_bt_ids */
} gsp_step_desc;

/* Validates and packs one engine step for `pool` (its KV-head count and
 * block count) and uploads it in one copy (a copy kernel that reads the
 * pinned staging buffer) on the context's stream; the packed step serves every layer of that pool.  Query
 * token i of row b sits at pos = positions[b] + i and attends to
 *     total = min(token_counts[b], pos + 1)           (PagedAttentionKernel.cs:41)
 * tokens (causal for q_lens[b] > 1, PagedTransformerRunner.cs:454-474); a row
 * whose every query token has total == 0 is skipped and its out rows are left
 * untouched (PagedAttentionKernel.cs:42).  Only the first ceil(total/block_size)
 * table entries of a row are packed.  Errors (GSP_E_INVALID_ARG):
 *   max_seq_len <= 0; pos < 0 or pos + q_len - 1 >= max_seq_len
 *   (PagedAttentionKernel.cs:34-37); token_counts[b] > max_seq_len (:38-39);
 *   bt_offsets outside [0, n_bt_ids] or decreasing; a row's table shorter
 *   than ceil(total/block_size); a block id outside the pool. */
int gsp_step_pack(gsp_ctx* ctx, const gsp_pool* pool, const gsp_step_desc* desc);

/* Sizes of the packed step (for tests and the bench). */
typedef struct gsp_step_info {
    int32_t num_rows;
    int32_t total_q;             /* query tokens in the step = sum of q_lens */
    int32_t packed_pages;        /* bt entries actually packed */
    int32_t heads_kv;            /* KV heads of the pool the step was packed for */
    int32_t decode_units;        /* (query, KV head, page range) units = decode workgroups */
    int32_t split_pairs;         /* (query, KV head) pairs cut into several units */
    int32_t partial_slots;       /* split partials written and merged */
    int32_t pages_per_split;     /* largest unit, in pages */
    int64_t kv_tokens;           /* sum over rows of the longest total (KV tokens read once) */
    int64_t staging_bytes;       /* bytes of the single host-to-device upload */
    int32_t prefill_tiles;       /* (16 query tokens, KV head) tiles of prefill rows */
    int32_t prefill_queries;     /* query tokens served by those tiles */
    int64_t prefill_pairs;       /* sum over tiled query tokens of total (causal key count) */
    int32_t decode_bins;         /* decode workgroups: each runs one bin of units back to back */
    int32_t split_records;       /* page-pair split records of fp32 tiles (0: the tiles split their pages) */
    int64_t pack_host_ns;        /* host time of the gsp_step_pack call that made the step:
                                    validation, scheduling, staging and the copy's enqueue */
    int64_t pack_wait_ns;        /* the part of pack_host_ns spent waiting for the staging
                                    slot: the upload that used it two packs earlier (and, after a
                                    capture read the slot, the context's stream) */
} gsp_step_info;

int gsp_step_get_info(const gsp_ctx* ctx, gsp_step_info* out);

/* Downloads the packed CSR table as it lives in device memory:
 * row_offsets[num_rows+1] and ids[packed_pages], plus ctx_lens[total_q] (the
 * `total` of each query token).  Any output may be NULL.  Synchronous. */
int gsp_step_download(gsp_ctx* ctx, int32_t* row_offsets, int32_t* ids, int32_t* ctx_lens);

/* Largest split-KV unit, in pages, for the next gsp_step_pack: 0 (default)
 * sizes units from the step's page count and the device's CU count; > 0
 * forces it (tuning and tests, e.g. 1 cuts every query token into one-page
 * splits).  A query token is never cut into more than 256 splits. */
int gsp_set_split_pages(gsp_ctx* ctx, int32_t pages);

/* Most decode workgroups for the next gsp_step_pack: 0 (default) uses two
 * per CU, or one per four CUs when the step also has prefill tiles (those run
 * beside the decode units, on a second stream forked from and joined back
 * into the context's stream); > 0 forces the count (tuning and tests).  Units
 * are packed into that many bins longest first, and each workgroup runs its
 * bin's units back to back. */
int gsp_set_decode_bins(gsp_ctx* ctx, int32_t bins);

/* Decode kernel selection (tuning and tests): GSP_DECODE_AUTO picks the
 * matrix-core kernel; GSP_DECODE_DPP forces the VALU/DPP kernel (GQA groups up
 * to 8); GSP_DECODE_MFMA forces the matrix-core kernel (groups up to 16). */
#define GSP_DECODE_AUTO 0
#define GSP_DECODE_DPP 1
#define GSP_DECODE_MFMA 2
int gsp_set_decode_path(gsp_ctx* ctx, int32_t path);

/* Prefill-row routing for the next gsp_step_pack (tuning and tests).
 * GSP_PREFILL_AUTO runs rows with q_len >= 16 as matrix-core tiles of 16 query
 * tokens x one KV head, which read each K/V page once per tile; shorter rows
 * go through the decode kernel one query token at a time.  GSP_PREFILL_TILES
 * tiles every row with q_len >= 2; GSP_PREFILL_PER_TOKEN tiles none. */
#define GSP_PREFILL_AUTO 0
#define GSP_PREFILL_TILES 1
#define GSP_PREFILL_PER_TOKEN 2
int gsp_set_prefill_path(gsp_ctx* ctx, int32_t path);

/* How prefill tiles over fp32 pages get the fp16 hi/lo split of the pages
 * they read, for the next gsp_step_pack (tuning and tests).
 * GSP_SPLIT_RECORDS (the default): gsp_attention_step first writes each page
 * pair of each tiled row and KV head once as a split record (a device
 * workspace of about 17 KB per page and KV head at head_dim 128, sized by
 * gsp_step_pack), and the tiles copy records into LDS.  GSP_SPLIT_IN_TILE:
 * every tile splits the pages it reads (no workspace; the form
 * gsp_attention_step_noalloc always uses).  Both give results within the
 * same bound; fp16 pools are not affected. */
#define GSP_SPLIT_RECORDS 0
#define GSP_SPLIT_IN_TILE 1
int gsp_set_prefill_split(gsp_ctx* ctx, int32_t mode);

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* PagedAttentionKernel.ComputeAttention (PagedAttentionKernel.cs:17-372)
 * over every query token of the packed step at once.
 *   q_dev   [total_q][n_heads][head_dim]  fp32, device
 *   out_dev [total_q][n_heads][v_head_dim] fp32, device
 * Query head h reads KV head h / (n_heads / heads_kv) (:44,50).  Scores are
 * dot(q, k) * attn_scale (:64-65), softmax over the row's `total` tokens (:70),
 * out = sum p_t v_t (:73-370).  sink_logit must be NULL: attention sinks are
 * unsupported on the GPU path, as in CudaPagedTransformerRunner.cs:431.
 * Supported, the domain of the reference GPU runner
 * (CudaPagedTransformerRunner.cs:402-412) and then some: head_dim and
 * v_head_dim from 1 to 256, odd ones included, and v_head_dim may differ from
 * head_dim, as in the CPU kernel's generic path (PagedAttentionKernel.cs:326-370); any
 * GQA group (n_heads % heads_kv == 0); pages of 1 to GSP_MAX_BLOCK_SIZE
 * tokens.  The kernels read pages of at most 16 tokens: a pool page of more
 * is read as equal parts of the largest size up to 16 that divides it (32 and
 * 64 as 16-token parts, 24 as 12, a prime size as single tokens).  The pool
 * must have the KV heads, block count and page size the step was packed for.
 * Rows with q_len >= 16 run as prefill tiles when head_dim == v_head_dim is 64
 * or 128 and the parts have 16 tokens, else as per-query decode units.
 * GSP_DECODE_DPP serves head_dim 64 or 128, 16-token parts and groups up to 8
 * only.  Work is
 * enqueued on the context's stream.  A step with both decode units and
 * prefill tiles runs them in one kernel (with GSP_DECODE_DPP: the tiles on
 * second streams of the context, forked from and joined back into that
 * stream, so the call is still ordered as a whole on the context's stream).
 *
 * Step uploads: gsp_step_pack alternates between two device slots and copies
 * the step with one copy kernel on the context's stream (it reads the pinned
 * host buffer over the bus), behind the kernels that read the slot's previous
 * step and before the kernels of the step; its pinned host buffer is
 * rewritten two packs later, once that copy is done.
 * Graph capture: the call can be captured on the context's stream once the
 * packed step's upload is known complete (gsp_sync after gsp_step_pack;
 * otherwise GSP_E_STATE).  gsp_step_pack sizes the split-KV workspace for
 * GQA groups up to 16 (it does not know n_heads); a larger group needs
 * ceil(group / 16) times that, which the first eager call with that group
 * allocates: run one before capturing (a captured call that would have to
 * grow the workspace fails with GSP_E_STATE and enqueues nothing).  The graph holds the step's kernels only and reads
 * the packed step's slot: it is valid until the next gsp_step_pack.  The pack
 * after that reuses the slot and first waits on the host for the context's
 * stream; replays launched on other streams must have finished by then. */
int gsp_attention_step(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads,
                       const float* q_dev, float* out_dev, float attn_scale,
                       const float* sink_logit);

/* Allocation-free variant of gsp_attention_step.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as gsp_attention_step, but the split-KV
 * workspace (partial outputs and per-(query, KV head) counters) lives in a
 * fixed device array of GSP_NOALLOC_SCRATCH_BYTES per GPU instead of context
 * memory: the call never allocates or frees, whatever the step's size.  Its
 * fp32 prefill tiles always split their own pages (GSP_SPLIT_IN_TILE), so its
 * results equal gsp_attention_step's bit for bit when the step was packed
 * with that mode, and within the fp32 bound otherwise.  The
 * array's first GSP_NOALLOC_COUNTERS int32 words are counters (a step may use
 * total_q * heads_kv of them) and the rest holds partials (a step uses
 * partial_slots * (n_heads / heads_kv) * (v_head_dim + 2) floats); a step that
 * needs more fails with GSP_E_INVALID_ARG before anything is enqueued.  Each
 * call clears the counters it uses with a kernel on the context's stream.
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (two contexts' streams, or threads)
 * race and must be ordered by the caller.  The packed step must come from an
 * earlier gsp_step_pack (which may allocate, and cannot be captured). */
#define GSP_NOALLOC_SCRATCH_BYTES (16u << 20)
#define GSP_NOALLOC_COUNTERS 65536u
int gsp_attention_step_noalloc(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads,
                               const float* q_dev, float* out_dev, float attn_scale,
                               const float* sink_logit);

/* Single-sequence drop-in for ComputeAttention with the reference's argument
 * list (PagedAttentionKernel.cs:17-32): the BlockTable is passed as its id span
 * plus TokenCount; head geometry must match the pool.  head_scores is not
 * needed (online softmax) and is ignored.  Packs a one-row step and runs
 * it; returns after enqueueing. */
int gsp_compute_attention(gsp_ctx* ctx, const gsp_pool* pool, int32_t stage_layer,
                          int32_t model_layer, int32_t pos, const float* q_dev, float* out_dev,
                          const int32_t* block_ids, int32_t n_block_ids, int32_t token_count,
                          int32_t n_heads, int32_t n_heads_kv, int32_t head_dim,
                          int32_t v_head_dim, float attn_scale, float* head_scores,
                          int32_t max_seq_len, const float* sink_logit);

/* ------------------------------------------------------------------------ */
/* Host metadata: the block-id half of PagedBlockPool and BlockTable         */
/* (PagedBlockPool.cs:112-121,178-299; BlockTable.cs:13-117).  Host-only,    */
/* no device work except the optional COW page copy.                         */
/* ------------------------------------------------------------------------ */

/* LIFO free stack seeded so the first allocation returns block 0
 * (PagedBlockPool.cs:116-120).  total_blocks < 1 or block_size < 1 ->
 * GSP_E_INVALID_ARG (:63-67). */
int gsp_block_allocator_create(int32_t total_blocks, int32_t block_size,
                               gsp_block_allocator** out);
void gsp_block_allocator_destroy(gsp_block_allocator* a);

/* Attaches a device pool so that copy-on-write forks copy page contents on the
 * device (PagedBlockPool.TryForkBlock, :332-342).  NULL detaches; without a
 * pool a fork only allocates, as the reference's metadata-only pool does.  The
 * pool must hold at least the allocator's blocks.  The allocator itself is
 * safe to use from several threads at once (a mutex-guarded free stack,
 * atomic refcounts and a guarded prefix map), as the reference's pool is. */
int gsp_block_allocator_attach_pool(gsp_block_allocator* a, gsp_ctx* ctx, gsp_pool* pool);

/* TryAllocateBlock (:178-189): 1 and *block_id on success, 0 and -1 if empty. */
int gsp_block_allocator_try_allocate(gsp_block_allocator* a, int32_t* block_id);
/* RetainBlock (:240-245): new refcount, or -1 with GSP_E_INVALID_ARG set. */
int gsp_block_allocator_retain(gsp_block_allocator* a, int32_t block_id);
/* ReleaseBlock (:251-279): remaining refcount; idempotent double free. */
int gsp_block_allocator_release(gsp_block_allocator* a, int32_t block_id);
int gsp_block_allocator_ref_count(const gsp_block_allocator* a, int32_t block_id);
int gsp_block_allocator_free_count(const gsp_block_allocator* a);
int gsp_block_allocator_total(const gsp_block_allocator* a);

/* Prefix cache (PagedBlockPool.cs:163-234).
 * gsp_prefix_hash: ComputePrefixHash (:168-172), the 64-bit XXH3 hash of the
 * n token ids' little-endian bytes seeded with the parent block's hash (0 for
 * the first block): the cumulative Merkle chain over full blocks.  Returns 0
 * with GSP_E_INVALID_ARG set for an invalid span.
 * gsp_block_allocator_find_prefix: TryFindPrefixBlock (:194-220).  1 and
 * *block_id, with the block's refcount raised by one, if a live block holds
 * the hash; 0 and -1 otherwise (also for hash 0).
 * gsp_block_allocator_bind_prefix: BindPrefixBlock (:225-234), the last
 * binding of a hash wins.  GSP_E_INVALID_ARG for an id outside the pool or a
 * zero hash.  Allocating a block clears its hash; freeing it removes its map
 * entry if the hash still maps to it (:263-271). */
uint64_t gsp_prefix_hash(uint64_t parent_hash, const int32_t* tokens, int32_t n);
/* The chain over n_blocks consecutive full blocks of block_size tokens, in one
 * call: out[i] = gsp_prefix_hash(i ? out[i-1] : parent_hash, block i), what
 * ContinuousBatchEngine.cs:223-263 computes block by block when it admits a
 * prompt. */
int gsp_prefix_hash_chain(uint64_t parent_hash, const int32_t* tokens, int32_t n_blocks, int32_t block_size,
                          uint64_t* out);
int gsp_block_allocator_find_prefix(gsp_block_allocator* a, uint64_t prefix_hash, int32_t* block_id);
int gsp_block_allocator_bind_prefix(gsp_block_allocator* a, uint64_t prefix_hash, int32_t block_id);

int gsp_block_table_create(gsp_block_allocator* a, gsp_block_table** out);
void gsp_block_table_destroy(gsp_block_table* t);
/* AttachPrefixBlocks (BlockTable.cs:31-39). */
int gsp_block_table_attach_prefix(gsp_block_table* t, const int32_t* ids, int32_t n,
                                  int32_t token_count);
/* AppendToken (BlockTable.cs:46-80): 1 on success, 0 on pool exhaustion with
 * the table unchanged and *block_id = *offset = -1.  -1 with GSP_E_INVALID_ARG
 * set (table unchanged) for a NULL argument, and where the reference throws:
 * TokenCount is inside a page but the table holds no page (an empty prefix
 * attached with a nonzero token count; `_physicalBlockIds[^1]`,
 * BlockTable.cs:60). */
int gsp_block_table_append_token(gsp_block_table* t, int32_t* block_id, int32_t* offset);
/* AppendToken n times, as a prefill chunk reserves its slots
 * (PagedTransformerRunner.cs:383-401); stops at the first failure.  Returns
 * the number of tokens appended. */
int gsp_block_table_append_tokens(gsp_block_table* t, int32_t n);
/* GetTokenLocation (BlockTable.cs:86-91). */
int gsp_block_table_token_location(const gsp_block_table* t, int32_t token, int32_t* block_id,
                                   int32_t* offset);
int gsp_block_table_block_id(const gsp_block_table* t, int32_t index);
int gsp_block_table_token_count(const gsp_block_table* t);
int gsp_block_table_block_count(const gsp_block_table* t);
/* AsSpan (BlockTable.cs:103): copies up to cap ids; returns the block count. */
int gsp_block_table_ids(const gsp_block_table* t, int32_t* out, int32_t cap);
/* ReleaseAll (BlockTable.cs:108-116). */
void gsp_block_table_release_all(gsp_block_table* t);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_PAGED_H */
