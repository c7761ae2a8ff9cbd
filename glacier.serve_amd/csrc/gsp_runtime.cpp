// Host runtime behind the C ABI of glacier_paged.h: device context, KV pool
// arenas in HBM, the per-step packer (one pinned staging buffer, one
// host-to-device copy) and kernel dispatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/glacier_paged.h"
#include "gsp_internal.h"
#include "gsp_status.h"

using gsp::DecodeUnit;
using gsp::MergeItem;

namespace {

// Packed step layout, in int32 elements from the start of the staging buffer.
enum : int {
    kHdrRows = 0,
    kHdrTotalQ,
    kHdrPages,
    kHdrUnits,
    kHdrSplitPages,
    kHdrSlots,
    kHdrMaxId,
    kHdrMerges,
    kHdrWords = 16
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool is_oom(hipError_t e) { return e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation; }

}  // namespace

struct gsp_ctx {
    int device = 0;
    int num_cus = 0;
    std::string arch;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;

    // Step staging: pinned host buffer, its device mirror, and an event that
    // marks when the last upload out of the staging buffer has completed.
    int32_t* staging = nullptr;
    size_t staging_words = 0;
    int32_t* d_step = nullptr;
    size_t d_step_words = 0;
    hipEvent_t staging_done = nullptr;
    bool staging_pending = false;

    // Auxiliary staging for pool writes.
    int32_t* aux = nullptr;
    size_t aux_words = 0;
    int32_t* d_aux = nullptr;
    size_t d_aux_words = 0;
    hipEvent_t aux_done = nullptr;
    bool aux_pending = false;

    // Packed-step metadata (host copy).
    bool step_valid = false;
    gsp_step_info info{};
    int32_t max_id = -1;
    size_t off_rows = 0, off_ids = 0, off_ctx = 0, off_units = 0, off_merge = 0;

    // Split-KV workspace.
    float* part = nullptr;
    size_t part_floats = 0;

    int32_t split_pages_override = 0;
    int32_t decode_path = GSP_DECODE_AUTO;
    int32_t num_slots = 0;   // partial slots of the packed step
    int32_t num_merges = 0;  // query tokens whose partials need merging

    // Host scratch reused across steps.
    std::vector<DecodeUnit> units;
    std::vector<MergeItem> merges;
    std::vector<int32_t> q_ctx;
};

struct gsp_pool {
    gsp_ctx* ctx = nullptr;
    gsp_pool_desc desc{};
    void* k = nullptr;
    void* v = nullptr;
    size_t k_bytes = 0, v_bytes = 0;
    bool owned = false;
    int64_t head_stride_k = 0, layer_stride_k = 0, block_stride_k = 0;
    int64_t head_stride_v = 0, layer_stride_v = 0, block_stride_v = 0;
};

namespace {

int elem_bytes(const gsp_pool_desc& d) { return d.kv_dtype == GSP_KV_F16 ? 2 : 4; }

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return GSP_OK;
    (void)hipGetLastError();
    if (is_oom(e)) return gsp::fail(GSP_E_OOM, "%s: %s", what, hipGetErrorString(e));
    return gsp::fail(GSP_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

int set_device(const gsp_ctx* ctx) { return check_hip(hipSetDevice(ctx->device), "hipSetDevice"); }

// Grows a pinned host buffer (waiting for the upload that last used it).
int ensure_pinned(int32_t** buf, size_t* cap, size_t words, hipEvent_t done, bool* pending) {
    if (*pending) {
        int rc = check_hip(hipEventSynchronize(done), "hipEventSynchronize(staging)");
        if (rc) return rc;
        *pending = false;
    }
    if (words <= *cap) return GSP_OK;
    size_t n = std::max(words, *cap * 2);
    if (*buf) (void)hipHostFree(*buf);
    *buf = nullptr;
    *cap = 0;
    int rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(buf), n * sizeof(int32_t),
                                     hipHostMallocDefault),
                       "hipHostMalloc(staging)");
    if (rc) return rc;
    *cap = n;
    return GSP_OK;
}

// Grows a device buffer.  The stream is synchronised first so no queued
// kernel still reads the old allocation.
template <typename T>
int ensure_device(gsp_ctx* ctx, T** buf, size_t* cap, size_t count, bool zero) {
    if (count <= *cap) return GSP_OK;
    int rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    size_t n = std::max(count, *cap * 2);
    if (*buf) (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
    rc = check_hip(hipMalloc(reinterpret_cast<void**>(buf), n * sizeof(T)), "hipMalloc(workspace)");
    if (rc) return rc;
    if (zero) {
        rc = check_hip(hipMemsetAsync(*buf, 0, n * sizeof(T), ctx->stream), "hipMemsetAsync");
        if (rc) return rc;
    }
    *cap = n;
    return GSP_OK;
}

// Pages per split-KV unit: enough units to give every CU about one
// workgroup per KV head, never fewer than one page per wave.
int32_t choose_split_pages(const gsp_ctx* ctx, int64_t total_pages) {
    if (ctx->split_pages_override > 0) return ctx->split_pages_override;
    int64_t cus = std::max(1, ctx->num_cus);
    int64_t pps = (total_pages + cus - 1) / cus;
    pps = (pps + gsp::kDecodeWaves - 1) / gsp::kDecodeWaves * gsp::kDecodeWaves;
    pps = std::max<int64_t>(gsp::kDecodeWaves, std::min<int64_t>(pps, 256));
    return static_cast<int32_t>(pps);
}

int validate_pool_desc(const gsp_pool_desc* d) {
    if (!d) return gsp::fail(GSP_E_INVALID_ARG, "pool descriptor is NULL");
    if (d->total_blocks < 1) return gsp::fail(GSP_E_INVALID_ARG, "totalBlocks must be >= 1 (got %d)", d->total_blocks);
    if (d->layers < 1) return gsp::fail(GSP_E_INVALID_ARG, "layers must be >= 1 (got %d)", d->layers);
    if (d->heads_kv < 1) return gsp::fail(GSP_E_INVALID_ARG, "headsKv must be >= 1 (got %d)", d->heads_kv);
    if (d->head_dim < 1) return gsp::fail(GSP_E_INVALID_ARG, "headDim must be >= 1 (got %d)", d->head_dim);
    if (d->block_size < 1) return gsp::fail(GSP_E_INVALID_ARG, "blockSize must be >= 1 (got %d)", d->block_size);
    if (d->kv_dtype != GSP_KV_F32 && d->kv_dtype != GSP_KV_F16)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown kv_dtype %d", d->kv_dtype);
    if (d->block_size != GSP_BLOCK_SIZE)
        return gsp::fail(GSP_E_UNSUPPORTED, "device pool supports blockSize 16 only (got %d)", d->block_size);
    return GSP_OK;
}

void fill_strides(gsp_pool* p) {
    const gsp_pool_desc& d = p->desc;
    p->head_stride_k = (int64_t)d.block_size * d.head_dim;
    p->layer_stride_k = (int64_t)d.heads_kv * p->head_stride_k;
    p->block_stride_k = (int64_t)d.layers * p->layer_stride_k;
    p->head_stride_v = (int64_t)d.block_size * d.v_head_dim;
    p->layer_stride_v = (int64_t)d.heads_kv * p->head_stride_v;
    p->block_stride_v = (int64_t)d.layers * p->layer_stride_v;
    p->k_bytes = (size_t)d.total_blocks * p->block_stride_k * elem_bytes(d);
    p->v_bytes = (size_t)d.total_blocks * p->block_stride_v * elem_bytes(d);
}

}  // namespace

extern "C" {

int gsp_abi_version(void) { return GSP_ABI_VERSION; }

int gsp_device_info_get(int device, gsp_device_info* out) {
    gsp::clear_error();
    if (!out) return gsp::fail(GSP_E_INVALID_ARG, "out is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return gsp::fail(GSP_E_UNSUPPORTED, "no HIP device available");
    }
    if (device < 0 || device >= n) return gsp::fail(GSP_E_INVALID_ARG, "device %d out of range [0, %d)", device, n);
    hipDeviceProp_t prop;
    int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (rc) return rc;
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    out->compute_units = prop.multiProcessorCount;
    out->wavefront_size = prop.warpSize;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width_bits = prop.memoryBusWidth;
    out->total_global_mem = (int64_t)prop.totalGlobalMem;
    out->lds_per_block = (int64_t)prop.sharedMemPerBlock;
    return GSP_OK;
}

int gsp_init(int device, gsp_ctx** out) {
    gsp::clear_error();
    if (!out) return gsp::fail(GSP_E_INVALID_ARG, "out is NULL");
    *out = nullptr;
    gsp_device_info info;
    int rc = gsp_device_info_get(device, &info);
    if (rc) return rc;
    if (std::strncmp(info.arch, "gfx950", 6) != 0)
        return gsp::fail(GSP_E_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only", device, info.arch);
    gsp_ctx* ctx = new gsp_ctx();
    ctx->device = device;
    ctx->num_cus = info.compute_units;
    ctx->arch = info.arch;
    rc = set_device(ctx);
    if (!rc) rc = check_hip(hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking), "hipStreamCreate");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&ctx->staging_done, hipEventDisableTiming), "hipEventCreate");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&ctx->aux_done, hipEventDisableTiming), "hipEventCreate");
    if (rc) {
        gsp_shutdown(ctx);
        return rc;
    }
    ctx->stream = ctx->own_stream;
    *out = ctx;
    return GSP_OK;
}

void gsp_shutdown(gsp_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->staging) (void)hipHostFree(ctx->staging);
    if (ctx->aux) (void)hipHostFree(ctx->aux);
    if (ctx->d_step) (void)hipFree(ctx->d_step);
    if (ctx->d_aux) (void)hipFree(ctx->d_aux);
    if (ctx->part) (void)hipFree(ctx->part);
    if (ctx->staging_done) (void)hipEventDestroy(ctx->staging_done);
    if (ctx->aux_done) (void)hipEventDestroy(ctx->aux_done);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    (void)hipGetLastError();
    delete ctx;
}

int gsp_set_stream(gsp_ctx* ctx, void* hip_stream) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    hipStream_t next = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    if (next != ctx->stream) {
        // Work already queued keeps its order relative to what follows.
        int rc = set_device(ctx);
        if (!rc) rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (rc) return rc;
    }
    ctx->stream = next;
    return GSP_OK;
}

void* gsp_get_stream(gsp_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int gsp_sync(gsp_ctx* ctx) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    int rc = set_device(ctx);
    if (rc) return rc;
    return check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int gsp_set_split_pages(gsp_ctx* ctx, int32_t pages) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (pages < 0) return gsp::fail(GSP_E_INVALID_ARG, "split pages must be >= 0 (got %d)", pages);
    ctx->split_pages_override = pages;
    return GSP_OK;
}

int gsp_set_decode_path(gsp_ctx* ctx, int32_t path) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (path != GSP_DECODE_AUTO && path != GSP_DECODE_DPP && path != GSP_DECODE_MFMA)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown decode path %d", path);
    ctx->decode_path = path;
    return GSP_OK;
}

/* ---------------------------------------------------------------- pools */

int gsp_pool_create(gsp_ctx* ctx, const gsp_pool_desc* desc, gsp_pool** out) {
    gsp::clear_error();
    if (!ctx || !out) return gsp::fail(GSP_E_INVALID_ARG, "ctx/out is NULL");
    *out = nullptr;
    int rc = validate_pool_desc(desc);
    if (rc) return rc;
    gsp_pool* p = new gsp_pool();
    p->ctx = ctx;
    p->desc = *desc;
    if (p->desc.v_head_dim <= 0) p->desc.v_head_dim = p->desc.head_dim;
    fill_strides(p);
    p->owned = true;
    rc = set_device(ctx);
    if (!rc) rc = check_hip(hipMalloc(&p->k, p->k_bytes), "hipMalloc(K pool)");
    if (!rc) rc = check_hip(hipMalloc(&p->v, p->v_bytes), "hipMalloc(V pool)");
    if (!rc) rc = check_hip(hipMemsetAsync(p->k, 0, p->k_bytes, ctx->stream), "hipMemsetAsync(K pool)");
    if (!rc) rc = check_hip(hipMemsetAsync(p->v, 0, p->v_bytes, ctx->stream), "hipMemsetAsync(V pool)");
    if (!rc) rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) {
        gsp_pool_destroy(p);
        return rc;
    }
    *out = p;
    return GSP_OK;
}

int gsp_pool_wrap(gsp_ctx* ctx, const gsp_pool_desc* desc, void* k_dev, void* v_dev, gsp_pool** out) {
    gsp::clear_error();
    if (!ctx || !out) return gsp::fail(GSP_E_INVALID_ARG, "ctx/out is NULL");
    *out = nullptr;
    int rc = validate_pool_desc(desc);
    if (rc) return rc;
    if (!k_dev || !v_dev) return gsp::fail(GSP_E_INVALID_ARG, "arena pointers must not be NULL");
    if ((reinterpret_cast<uintptr_t>(k_dev) | reinterpret_cast<uintptr_t>(v_dev)) & 15)
        return gsp::fail(GSP_E_INVALID_ARG, "arenas must be 16-byte aligned");
    gsp_pool* p = new gsp_pool();
    p->ctx = ctx;
    p->desc = *desc;
    if (p->desc.v_head_dim <= 0) p->desc.v_head_dim = p->desc.head_dim;
    fill_strides(p);
    p->k = k_dev;
    p->v = v_dev;
    p->owned = false;
    *out = p;
    return GSP_OK;
}

void gsp_pool_destroy(gsp_pool* pool) {
    if (!pool) return;
    if (pool->owned) {
        (void)hipSetDevice(pool->ctx->device);
        (void)hipStreamSynchronize(pool->ctx->stream);
        if (pool->k) (void)hipFree(pool->k);
        if (pool->v) (void)hipFree(pool->v);
        (void)hipGetLastError();
    }
    delete pool;
}

int gsp_pool_arenas(const gsp_pool* pool, void** k_dev, void** v_dev, size_t* k_bytes, size_t* v_bytes) {
    gsp::clear_error();
    if (!pool) return gsp::fail(GSP_E_INVALID_ARG, "pool is NULL");
    if (k_dev) *k_dev = pool->k;
    if (v_dev) *v_dev = pool->v;
    if (k_bytes) *k_bytes = pool->k_bytes;
    if (v_bytes) *v_bytes = pool->v_bytes;
    return GSP_OK;
}

int gsp_pool_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* block_ids,
                          const int32_t* slots, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (n < 0) return gsp::fail(GSP_E_INVALID_ARG, "n must be >= 0 (got %d)", n);
    if (n == 0) return GSP_OK;
    if (!block_ids || !slots || !k_dev || !v_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    const gsp_pool_desc& d = pool->desc;
    if (d.v_head_dim != d.head_dim) return gsp::fail(GSP_E_UNSUPPORTED, "vHeadDim != headDim is not supported on the device pool");
    if (layer < 0 || layer >= d.layers) return gsp::fail(GSP_E_INVALID_ARG, "layer %d out of range [0, %d)", layer, d.layers);
    for (int32_t i = 0; i < n; ++i) {
        if (block_ids[i] < 0 || block_ids[i] >= d.total_blocks)
            return gsp::fail(GSP_E_INVALID_ARG, "block id %d out of range [0, %d)", block_ids[i], d.total_blocks);
        if (slots[i] < 0 || slots[i] >= d.block_size)
            return gsp::fail(GSP_E_INVALID_ARG, "slot %d out of range [0, %d)", slots[i], d.block_size);
    }
    int rc = set_device(ctx);
    if (rc) return rc;
    const size_t words = 2 * (size_t)n;
    rc = ensure_pinned(&ctx->aux, &ctx->aux_words, words, ctx->aux_done, &ctx->aux_pending);
    if (!rc) rc = ensure_device(ctx, &ctx->d_aux, &ctx->d_aux_words, words, false);
    if (rc) return rc;
    std::memcpy(ctx->aux, block_ids, n * sizeof(int32_t));
    std::memcpy(ctx->aux + n, slots, n * sizeof(int32_t));
    rc = check_hip(hipMemcpyAsync(ctx->d_aux, ctx->aux, words * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream),
                   "hipMemcpyAsync(write ids)");
    if (!rc) rc = check_hip(hipEventRecord(ctx->aux_done, ctx->stream), "hipEventRecord");
    if (rc) return rc;
    ctx->aux_pending = true;
    gsp::WriteTokensArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.block_ids = ctx->d_aux;
    a.slots = ctx->d_aux + n;
    a.k = k_dev;
    a.v = v_dev;
    a.n = n;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    return check_hip(gsp::launch_write_tokens(d.kv_dtype == GSP_KV_F16, a, ctx->stream), "write_tokens launch");
}

int gsp_pool_copy_block(gsp_ctx* ctx, gsp_pool* pool, int32_t src, int32_t dst, int32_t valid_tokens) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    const gsp_pool_desc& d = pool->desc;
    if (src < 0 || src >= d.total_blocks || dst < 0 || dst >= d.total_blocks)
        return gsp::fail(GSP_E_INVALID_ARG, "block ids (%d, %d) out of range [0, %d)", src, dst, d.total_blocks);
    if (valid_tokens <= 0) return GSP_OK;
    if (d.v_head_dim != d.head_dim) return gsp::fail(GSP_E_UNSUPPORTED, "vHeadDim != headDim is not supported on the device pool");
    int rc = set_device(ctx);
    if (rc) return rc;
    gsp::CopyBlockArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.head_stride = pool->head_stride_k;
    a.src = src;
    a.dst = dst;
    a.valid_tokens = std::min(valid_tokens, d.block_size);
    a.layers = d.layers;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    return check_hip(gsp::launch_copy_block(d.kv_dtype == GSP_KV_F16, a, ctx->stream), "copy_block launch");
}

static int pool_copy(gsp_ctx* ctx, gsp_pool* pool, int32_t which, size_t offset, void* host, size_t bytes,
                     bool upload) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (which != 0 && which != 1) return gsp::fail(GSP_E_INVALID_ARG, "which must be 0 (K) or 1 (V)");
    size_t cap = which == 0 ? pool->k_bytes : pool->v_bytes;
    if (offset > cap || bytes > cap - offset)
        return gsp::fail(GSP_E_INVALID_ARG, "range [%zu, %zu) exceeds the arena (%zu bytes)", offset, offset + bytes, cap);
    if (bytes == 0) return GSP_OK;
    if (!host) return gsp::fail(GSP_E_INVALID_ARG, "host pointer is NULL");
    int rc = set_device(ctx);
    if (rc) return rc;
    char* dev = static_cast<char*>(which == 0 ? pool->k : pool->v) + offset;
    rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    if (upload)
        return check_hip(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice), "hipMemcpy(upload)");
    return check_hip(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost), "hipMemcpy(download)");
}

int gsp_pool_upload(gsp_ctx* ctx, gsp_pool* pool, int32_t which, size_t offset_bytes, const void* host,
                    size_t bytes) {
    return pool_copy(ctx, pool, which, offset_bytes, const_cast<void*>(host), bytes, true);
}

int gsp_pool_download(gsp_ctx* ctx, gsp_pool* pool, int32_t which, size_t offset_bytes, void* host, size_t bytes) {
    return pool_copy(ctx, pool, which, offset_bytes, host, bytes, false);
}

/* ---------------------------------------------------------------- steps */

int gsp_step_pack(gsp_ctx* ctx, const gsp_step_desc* desc) {
    gsp::clear_error();
    if (!ctx || !desc) return gsp::fail(GSP_E_INVALID_ARG, "ctx/desc is NULL");
    ctx->step_valid = false;
    const int32_t B = desc->num_rows;
    if (B < 0) return gsp::fail(GSP_E_INVALID_ARG, "num_rows must be >= 0 (got %d)", B);
    if (desc->max_seq_len <= 0)
        return gsp::fail(GSP_E_INVALID_ARG, "maxSeqLen must be positive (got %d)", desc->max_seq_len);
    if (B > 0 && (!desc->positions || !desc->token_counts || !desc->bt_offsets || !desc->bt_ids))
        return gsp::fail(GSP_E_INVALID_ARG, "positions/token_counts/bt_offsets/bt_ids must not be NULL");
    const int32_t L = desc->max_seq_len;

    // Pass 1: validate rows and size the packed arrays.
    int64_t total_q = 0, packed_pages = 0, kv_tokens = 0, unit_pages = 0;
    if (B > 0 && desc->bt_offsets[0] < 0)
        return gsp::fail(GSP_E_INVALID_ARG, "bt_offsets[0] must be >= 0");
    for (int32_t b = 0; b < B; ++b) {
        const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
        const int32_t pos = desc->positions[b];
        const int32_t tc = desc->token_counts[b];
        if (ql < 0) return gsp::fail(GSP_E_INVALID_ARG, "row %d: q_len must be >= 0 (got %d)", b, ql);
        const int64_t last = (int64_t)pos + std::max(ql, 1) - 1;
        if (pos < 0 || last >= L)
            return gsp::fail(GSP_E_INVALID_ARG, "row %d: token position %lld exceeds valid sequence range [0, %d]", b,
                             (long long)(pos < 0 ? pos : last), L - 1);
        if (tc < 0) return gsp::fail(GSP_E_INVALID_ARG, "row %d: token count %d is negative", b, tc);
        if (tc > L) return gsp::fail(GSP_E_INVALID_ARG, "row %d: BlockTable token count %d exceeds maxSeqLen %d", b, tc, L);
        const int32_t span = desc->bt_offsets[b + 1] - desc->bt_offsets[b];
        if (span < 0) return gsp::fail(GSP_E_INVALID_ARG, "row %d: bt_offsets decrease", b);
        const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
        const int64_t pages = (total_last + gsp::kBlockSize - 1) / gsp::kBlockSize;
        if (pages > span)
            return gsp::fail(GSP_E_INVALID_ARG, "row %d: %lld tokens need %lld blocks but the table holds %d", b,
                             (long long)total_last, (long long)pages, span);
        const int32_t* ids = desc->bt_ids + desc->bt_offsets[b];
        for (int64_t i = 0; i < pages; ++i)
            if (ids[i] < 0) return gsp::fail(GSP_E_INVALID_ARG, "row %d: block id %d is negative", b, ids[i]);
        total_q += ql;
        packed_pages += pages;
        kv_tokens += total_last;
        for (int32_t i = 0; i < ql; ++i) {
            const int64_t tot = std::min<int64_t>(tc, (int64_t)pos + i + 1);
            unit_pages += (tot + gsp::kBlockSize - 1) / gsp::kBlockSize;
        }
    }
    if (total_q > INT32_MAX / 4 || packed_pages > INT32_MAX / 4)
        return gsp::fail(GSP_E_INVALID_ARG, "step too large");

    // Pass 2: per-query contexts and split-KV units.
    const int32_t pps = choose_split_pages(ctx, unit_pages);
    ctx->units.clear();
    ctx->merges.clear();
    ctx->q_ctx.assign((size_t)total_q, 0);
    int64_t slots = 0;
    {
        int64_t qi = 0, bt_base = 0;
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
            const int32_t pos = desc->positions[b];
            const int32_t tc = desc->token_counts[b];
            const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
            for (int32_t i = 0; i < ql; ++i, ++qi) {
                const int32_t tot = (int32_t)std::min<int64_t>(tc, (int64_t)pos + i + 1);
                ctx->q_ctx[qi] = tot;
                if (tot <= 0) continue;
                const int32_t pages = (tot + gsp::kBlockSize - 1) / gsp::kBlockSize;
                const int32_t nsplit = (pages + pps - 1) / pps;
                for (int32_t s = 0; s < nsplit; ++s) {
                    DecodeUnit u;
                    u.qi = (int32_t)qi;
                    u.bt_base = (int32_t)bt_base;
                    u.page_begin = s * pps;
                    u.page_end = std::min(pages, (s + 1) * pps);
                    u.ctx = tot;
                    u.split = s;
                    u.nsplit = nsplit;
                    u.slot = nsplit > 1 ? (int32_t)slots : 0;
                    ctx->units.push_back(u);
                }
                if (nsplit > 1) {
                    ctx->merges.push_back(MergeItem{(int32_t)qi, (int32_t)slots, nsplit, 0});
                    slots += nsplit;
                }
            }
            bt_base += (total_last + gsp::kBlockSize - 1) / gsp::kBlockSize;
        }
    }
    // Longest units first so the tail of the grid is made of short ones.
    std::stable_sort(ctx->units.begin(), ctx->units.end(), [](const DecodeUnit& x, const DecodeUnit& y) {
        return (x.page_end - x.page_begin) > (y.page_end - y.page_begin);
    });

    // Pass 3: write the staging buffer.
    const size_t n_units = ctx->units.size();
    size_t off = kHdrWords;
    const size_t off_rows = off;
    off += (size_t)B + 1;
    const size_t off_ids = off;
    off += (size_t)packed_pages;
    const size_t off_ctx = off;
    off += (size_t)total_q;
    off = align_up(off, 8);
    const size_t off_units = off;
    off += n_units * (sizeof(DecodeUnit) / sizeof(int32_t));
    const size_t n_merges = ctx->merges.size();
    const size_t off_merge = off;
    off += n_merges * (sizeof(MergeItem) / sizeof(int32_t));
    const size_t words = off;

    int rc = set_device(ctx);
    if (rc) return rc;
    rc = ensure_pinned(&ctx->staging, &ctx->staging_words, words, ctx->staging_done, &ctx->staging_pending);
    if (!rc) rc = ensure_device(ctx, &ctx->d_step, &ctx->d_step_words, words, false);
    if (rc) return rc;

    int32_t* st = ctx->staging;
    std::memset(st, 0, kHdrWords * sizeof(int32_t));
    int32_t max_id = -1;
    {
        int32_t* rows = st + off_rows;
        int32_t* ids = st + off_ids;
        int64_t w = 0;
        rows[0] = 0;
        for (int32_t b = 0; b < B; ++b) {
            const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
            const int64_t total_last =
                ql > 0 ? std::min<int64_t>(desc->token_counts[b], (int64_t)desc->positions[b] + ql) : 0;
            const int64_t pages = (total_last + gsp::kBlockSize - 1) / gsp::kBlockSize;
            const int32_t* src = desc->bt_ids + desc->bt_offsets[b];
            for (int64_t i = 0; i < pages; ++i) {
                ids[w++] = src[i];
                max_id = std::max(max_id, src[i]);
            }
            rows[b + 1] = (int32_t)w;
        }
    }
    if (total_q) std::memcpy(st + off_ctx, ctx->q_ctx.data(), (size_t)total_q * sizeof(int32_t));
    if (n_units) std::memcpy(st + off_units, ctx->units.data(), n_units * sizeof(DecodeUnit));
    if (n_merges) std::memcpy(st + off_merge, ctx->merges.data(), n_merges * sizeof(MergeItem));
    st[kHdrRows] = B;
    st[kHdrTotalQ] = (int32_t)total_q;
    st[kHdrPages] = (int32_t)packed_pages;
    st[kHdrUnits] = (int32_t)n_units;
    st[kHdrSplitPages] = pps;
    st[kHdrSlots] = (int32_t)slots;
    st[kHdrMaxId] = max_id;
    st[kHdrMerges] = (int32_t)n_merges;

    rc = check_hip(hipMemcpyAsync(ctx->d_step, st, words * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream),
                   "hipMemcpyAsync(step)");
    if (!rc) rc = check_hip(hipEventRecord(ctx->staging_done, ctx->stream), "hipEventRecord");
    if (rc) return rc;
    ctx->staging_pending = true;

    ctx->off_rows = off_rows;
    ctx->off_ids = off_ids;
    ctx->off_ctx = off_ctx;
    ctx->off_units = off_units;
    ctx->off_merge = off_merge;
    ctx->max_id = max_id;
    ctx->num_slots = (int32_t)slots;
    ctx->num_merges = (int32_t)n_merges;
    ctx->info.num_rows = B;
    ctx->info.total_q = (int32_t)total_q;
    ctx->info.packed_pages = (int32_t)packed_pages;
    ctx->info.decode_units = (int32_t)n_units;
    ctx->info.prefill_tiles = 0;
    ctx->info.pages_per_split = pps;
    ctx->info.kv_tokens = kv_tokens;
    ctx->info.staging_bytes = (int64_t)(words * sizeof(int32_t));
    ctx->step_valid = true;
    return GSP_OK;
}

int gsp_step_get_info(const gsp_ctx* ctx, gsp_step_info* out) {
    gsp::clear_error();
    if (!ctx || !out) return gsp::fail(GSP_E_INVALID_ARG, "ctx/out is NULL");
    if (!ctx->step_valid) return gsp::fail(GSP_E_STATE, "no packed step");
    *out = ctx->info;
    return GSP_OK;
}

int gsp_step_download(gsp_ctx* ctx, int32_t* row_offsets, int32_t* ids, int32_t* ctx_lens) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (!ctx->step_valid) return gsp::fail(GSP_E_STATE, "no packed step");
    int rc = set_device(ctx);
    if (!rc) rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    const gsp_step_info& in = ctx->info;
    if (row_offsets)
        rc = check_hip(hipMemcpy(row_offsets, ctx->d_step + ctx->off_rows, ((size_t)in.num_rows + 1) * sizeof(int32_t),
                                 hipMemcpyDeviceToHost),
                       "hipMemcpy(rows)");
    if (!rc && ids && in.packed_pages)
        rc = check_hip(hipMemcpy(ids, ctx->d_step + ctx->off_ids, (size_t)in.packed_pages * sizeof(int32_t),
                                 hipMemcpyDeviceToHost),
                       "hipMemcpy(ids)");
    if (!rc && ctx_lens && in.total_q)
        rc = check_hip(hipMemcpy(ctx_lens, ctx->d_step + ctx->off_ctx, (size_t)in.total_q * sizeof(int32_t),
                                 hipMemcpyDeviceToHost),
                       "hipMemcpy(ctx)");
    return rc;
}

/* ------------------------------------------------------------ attention */

int gsp_attention_step(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads, const float* q_dev,
                       float* out_dev, float attn_scale, const float* sink_logit) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (!ctx->step_valid) return gsp::fail(GSP_E_STATE, "gsp_step_pack must succeed before gsp_attention_step");
    const gsp_pool_desc& d = pool->desc;
    if (sink_logit) return gsp::fail(GSP_E_UNSUPPORTED, "attention sinks are not supported on the GPU path");
    if (d.v_head_dim != d.head_dim)
        return gsp::fail(GSP_E_UNSUPPORTED, "vHeadDim (%d) != headDim (%d) is not supported", d.v_head_dim, d.head_dim);
    if (d.head_dim != 64 && d.head_dim != 128)
        return gsp::fail(GSP_E_UNSUPPORTED, "headDim %d is not supported (64 or 128)", d.head_dim);
    if (layer < 0 || layer >= d.layers) return gsp::fail(GSP_E_INVALID_ARG, "layer %d out of range [0, %d)", layer, d.layers);
    if (n_heads < 1 || n_heads % d.heads_kv != 0)
        return gsp::fail(GSP_E_INVALID_ARG, "nHeads (%d) must be a positive multiple of nHeadsKv (%d)", n_heads, d.heads_kv);
    const int group = n_heads / d.heads_kv;
    // The matrix-core kernel serves groups up to its 16-wide tile; the DPP
    // kernel is kept for explicit selection (groups up to 8).
    const bool use_mfma = ctx->decode_path == GSP_DECODE_MFMA ||
                          (ctx->decode_path == GSP_DECODE_AUTO && group <= gsp::kMaxGroupMfma);
    const int max_group = use_mfma ? gsp::kMaxGroupMfma : gsp::kMaxGroup;
    if (group > max_group)
        return gsp::fail(GSP_E_UNSUPPORTED, "GQA group %d exceeds %d query heads per KV head", group, max_group);
    if (ctx->max_id >= d.total_blocks)
        return gsp::fail(GSP_E_INVALID_ARG, "block id %d out of range [0, %d)", ctx->max_id, d.total_blocks);
    const gsp_step_info& in = ctx->info;
    if (in.decode_units == 0) return GSP_OK;
    if (!q_dev || !out_dev) return gsp::fail(GSP_E_INVALID_ARG, "q/out must not be NULL");
    int rc = set_device(ctx);
    if (rc) return rc;

    const int32_t slots = ctx->num_slots;
    if (slots > 0) {
        const size_t per_slot = (size_t)n_heads * (d.head_dim + 2);
        rc = ensure_device(ctx, &ctx->part, &ctx->part_floats, (size_t)slots * per_slot, false);
        if (rc) return rc;
    }

    gsp::DecodeArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.units = reinterpret_cast<const DecodeUnit*>(ctx->d_step + ctx->off_units);
    a.bt_ids = ctx->d_step + ctx->off_ids;
    a.q = q_dev;
    a.out = out_dev;
    a.part_o = ctx->part;
    a.part_ml = ctx->part ? ctx->part + (size_t)slots * n_heads * d.head_dim : nullptr;
    a.n_heads = n_heads;
    a.n_kv = d.heads_kv;
    a.scale_log2 = attn_scale * 1.4426950408889634f;
    const int f16 = d.kv_dtype == GSP_KV_F16;
    rc = use_mfma ? check_hip(gsp::launch_decode_mfma(d.head_dim, f16, in.decode_units, a, ctx->stream),
                              "decode (mfma) launch")
                  : check_hip(gsp::launch_decode(d.head_dim, f16, group, in.decode_units, a, ctx->stream),
                              "decode (dpp) launch");
    if (rc || ctx->num_merges == 0) return rc;
    gsp::MergeArgs m;
    m.items = reinterpret_cast<const MergeItem*>(ctx->d_step + ctx->off_merge);
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.out = out_dev;
    m.n_heads = n_heads;
    m.n_kv = d.heads_kv;
    return check_hip(gsp::launch_merge(d.head_dim, ctx->num_merges, m, ctx->stream), "merge launch");
}

int gsp_compute_attention(gsp_ctx* ctx, const gsp_pool* pool, int32_t stage_layer, int32_t model_layer, int32_t pos,
                          const float* q_dev, float* out_dev, const int32_t* block_ids, int32_t n_block_ids,
                          int32_t token_count, int32_t n_heads, int32_t n_heads_kv, int32_t head_dim,
                          int32_t v_head_dim, float attn_scale, float* head_scores, int32_t max_seq_len,
                          const float* sink_logit) {
    (void)model_layer;  // unused by the reference as well (PagedAttentionKernel.cs:19)
    (void)head_scores;  // the online softmax needs no score scratch
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    const gsp_pool_desc& d = pool->desc;
    if (n_heads_kv != d.heads_kv || head_dim != d.head_dim || v_head_dim != d.v_head_dim)
        return gsp::fail(GSP_E_INVALID_ARG, "head geometry (%d kv, d=%d, dv=%d) does not match the pool (%d, %d, %d)",
                         n_heads_kv, head_dim, v_head_dim, d.heads_kv, d.head_dim, d.v_head_dim);
    if (n_block_ids < 0 || (n_block_ids > 0 && !block_ids))
        return gsp::fail(GSP_E_INVALID_ARG, "block table span is invalid");
    int32_t offsets[2] = {0, n_block_ids};
    int32_t one = 1;
    static const int32_t empty_ids[1] = {0};
    gsp_step_desc s;
    s.num_rows = 1;
    s.max_seq_len = max_seq_len;
    s.positions = &pos;
    s.q_lens = &one;
    s.token_counts = &token_count;
    s.bt_offsets = offsets;
    s.bt_ids = n_block_ids ? block_ids : empty_ids;
    int rc = gsp_step_pack(ctx, &s);
    if (rc) return rc;
    return gsp_attention_step(ctx, pool, stage_layer, n_heads, q_dev, out_dev, attn_scale, sink_logit);
}

}  // extern "C"
