// Host runtime behind the C ABI of glacier_paged.h: device context, KV pool
// arenas in HBM, the per-step packer (one pinned staging buffer, one
// host-to-device copy) and kernel dispatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "../../include/glacier_paged.h"
#include "gsp_host_meta.h"
#include "gsp_internal.h"
#include "gsp_status.h"
#include "gsp_step_plan.h"

using gsp::DecodeUnit;
using gsp::PrefillTile;
namespace {

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool is_oom(hipError_t e) { return e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation; }

}  // namespace

struct gsp_ctx {
    int device = 0;
    int num_cus = 0;
    std::string arch;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // A step with both decode units and prefill tiles runs the decode kernel
    // on side_stream[0] and the tiles on side_stream[1], forked from `stream`
    // and joined back into it with the events.  Streams share the device's
    // few hardware queues (4 by default) in creation order, so a stream the
    // caller made may share a queue with either; the two side streams are
    // created one after the other and so take different queues, and the two
    // kernels run side by side whatever `stream` is.
    hipStream_t side_stream[2] = {nullptr, nullptr};
    hipEvent_t fork_ev = nullptr;
    hipEvent_t join_ev[2] = {nullptr, nullptr};

    // Step staging, double-buffered: successive packs alternate between two
    // slots, each a pinned host buffer and its device mirror.  A step's upload
    // is one copy kernel on the context's stream (upload_step_kernel, reading
    // the fine-grained pinned buffer over the bus), so stream order puts it
    // after the kernels that read the slot's previous step and before the
    // kernels of this one; no event crosses streams.  upload_done (recorded
    // after the copy) tells the host when the pinned buffer may be written
    // again: the pack two steps later usually finds it done, since the GPU is
    // at most a step behind.
    static constexpr int kSlots = 2;
    int32_t* staging[kSlots] = {};
    size_t staging_words[kSlots] = {};
    const void* staging_dev[kSlots] = {};  // staging[j] as the device addresses it
    int32_t* d_step_slot[kSlots] = {};
    size_t d_step_words[kSlots] = {};
    hipEvent_t upload_done[kSlots] = {};
    bool upload_pending[kSlots] = {};
    // The host has seen the slot's upload complete (gsp_sync): only then may
    // a graph capture read the slot, since a capture takes no event nodes.
    bool upload_synced[kSlots] = {};
    // A capture read the slot: its next upload first waits for the context's
    // stream on the host, where the graph's replays normally run.
    bool slot_captured[kSlots] = {};
    int slot = 0;               // slot of the packed step
    int32_t* d_step = nullptr;  // d_step_slot[slot]

    // Auxiliary staging for pool writes.
    int32_t* aux = nullptr;
    size_t aux_words = 0;
    int32_t* d_aux = nullptr;
    size_t d_aux_words = 0;
    // Split-K partials of gsp_matmul_batch, and x as fp16 pairs with row exponents (Q8_0).
    float* d_mm = nullptr;
    size_t d_mm_floats = 0;
    uint16_t* d_mmx = nullptr;
    size_t d_mmx_halves = 0;
    int32_t* d_mmexp = nullptr;
    size_t d_mmexp_words = 0;
    int32_t* d_mmcnt = nullptr;  // small-batch form: per-tile counters, zero between launches
    size_t d_mmcnt_words = 0;
    float* d_mmxs = nullptr;  // small-batch Q4_K: block sums of the scaled x
    size_t d_mmxs_floats = 0;
    hipEvent_t aux_done = nullptr;
    bool aux_pending = false;

    // Packed-step metadata (host copy).
    bool step_valid = false;
    gsp_step_info info{};
    int32_t max_id = -1;
    size_t off_rows = 0, off_ids = 0, off_ctx = 0, off_wr = 0, off_units = 0, off_tiles = 0, off_bins = 0;
    size_t off_split = 0;
    int32_t num_units = 0;      // decode units of the packed step
    int32_t num_bins = 0;       // decode workgroups (bins of units) of the packed step
    int32_t num_tiles = 0;      // prefill tiles of the packed step
    int32_t num_slots = 0;      // partial slots of the packed step
    int32_t step_heads_kv = 0;  // pool geometry the step was packed for
    int32_t step_blocks = 0;
    int32_t step_block_size = 0;
    int32_t step_page_tokens = 0;  // tokens per kernel page (the pool's page, or a part of it above 16)
    int32_t step_tile_pages = 1;   // kernel pages per decode tile (the units count tiles)
    bool step_tileable = false;
    // Split records of the packed step's fp32 prefill tiles (records_head_dim
    // 0: none, the tiles split their pages themselves): one per page pair of
    // each tiled row and KV head, written by gsp_attention_step per layer.
    int32_t num_split_items = 0;
    int32_t split_max_pairs = 0;
    int64_t num_records = 0;
    int32_t records_head_dim = 0;
    unsigned char* d_records = nullptr;
    size_t d_records_bytes = 0;

    // Split-KV workspace: partials and per-(query, KV head) split counters.
    float* part = nullptr;
    size_t part_floats = 0;
    int32_t* counters = nullptr;
    size_t counter_words = 0;

    int32_t split_pages_override = 0;
    int32_t decode_bins_override = 0;
    int32_t decode_path = GSP_DECODE_AUTO;
    int32_t prefill_path = GSP_PREFILL_AUTO;
    int32_t prefill_split = GSP_SPLIT_RECORDS;

    // The host packer and the plan of the packed step (its image, copied into
    // the pinned slot, and the sizes the launches need).
    gsp::StepPlanner planner;
    gsp::StepPlan plan;

    // RoPE angle-rate tables (gsp_rope_write_*_ex with inv_freq or
    // freq_factors): kRopeTables entries of kRopeMaxHalf doubles in one device
    // buffer, matched by content.  A new table takes the entry used least
    // recently; its copy runs on the context's stream from the pinned
    // staging, which rope_done guards.
    static constexpr int kRopeTables = 16;
    double* d_rope = nullptr;
    size_t d_rope_count = 0;
    int32_t* rope_staging = nullptr;
    size_t rope_staging_words = 0;
    hipEvent_t rope_done = nullptr;
    bool rope_pending = false;
    std::vector<double> rope_rates[kRopeTables];
    uint64_t rope_used[kRopeTables] = {};
    uint64_t rope_clock = 0;
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

// Whether `stream` is capturing into a graph.  Nothing may then allocate,
// free, synchronise or stage host memory on it.
int is_capturing(hipStream_t stream, bool* out) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const int rc = check_hip(hipStreamIsCapturing(stream, &st), "hipStreamIsCapturing");
    *out = rc == GSP_OK && st != hipStreamCaptureStatusNone;
    return rc;
}

// Kernels of the packed step read its device slot, which its upload wrote
// earlier on the same stream.  A graph capture needs the upload complete on
// the host already (gsp_sync after gsp_step_pack): the captured kernels run
// at replay time, long after the copy that preceded the capture.  It marks
// the slot so that the slot's next upload first drains the context's stream,
// where the replays run.
int step_begin(gsp_ctx* ctx, bool* capturing) {
    int rc = is_capturing(ctx->stream, capturing);
    if (rc) return rc;
    if (*capturing) {
        if (!ctx->upload_synced[ctx->slot])
            return gsp::fail(GSP_E_STATE,
                             "the packed step's upload is not known to be complete: call gsp_sync after "
                             "gsp_step_pack and before capturing");
        ctx->slot_captured[ctx->slot] = true;
    }
    return GSP_OK;
}

int step_done(gsp_ctx*, bool) { return GSP_OK; }

// Waits on the host for `ev`, spinning on the query first: a sleeping wait can
// add milliseconds to a step that is only microseconds behind.
int host_wait(hipEvent_t ev, const char* what) {
    for (int i = 0; i < 200000; ++i) {
        const hipError_t e = hipEventQuery(ev);
        if (e == hipSuccess) return GSP_OK;
        if (e != hipErrorNotReady) return check_hip(e, what);
    }
    return check_hip(hipEventSynchronize(ev), what);
}

// Grows a pinned host buffer (waiting for the upload that last used it).
// `flags` are hipHostMalloc's.
int ensure_pinned(int32_t** buf, size_t* cap, size_t words, hipEvent_t done, bool* pending,
                  unsigned flags = hipHostMallocDefault) {
    if (*pending) {
        int rc = host_wait(done, "hipEventSynchronize(staging)");
        if (rc) return rc;
        *pending = false;
    }
    if (words <= *cap) return GSP_OK;
    size_t n = std::max(words, *cap * 2);
    if (*buf) (void)hipHostFree(*buf);
    *buf = nullptr;
    *cap = 0;
    int rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(buf), n * sizeof(int32_t), flags),
                       "hipHostMalloc(staging)");
    if (rc) return rc;
    *cap = n;
    return GSP_OK;
}

// Grows a device buffer.  The stream is synchronised first so no queued
// kernel still reads the old allocation.  A stream that is capturing into a
// graph cannot do that: the call then fails with GSP_E_STATE, and the buffer
// must be grown by an eager call first (gsp_step_pack sizes the attention
// workspace for every group up to 16).  `zero` clears the new buffer with a
// kernel on the stream.
template <typename T>
int ensure_device(gsp_ctx* ctx, T** buf, size_t* cap, size_t count, bool zero) {
    if (count <= *cap) return GSP_OK;
    bool cap_on = false;
    int rc = is_capturing(ctx->stream, &cap_on);
    if (rc) return rc;
    if (cap_on)
        return gsp::fail(GSP_E_STATE,
                         "device workspace must grow to %zu bytes, which cannot happen while the stream is "
                         "capturing: run the same call once outside the capture first",
                         count * sizeof(T));
    rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    size_t n = std::max(count, *cap * 2);
    if (*buf) (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
    rc = check_hip(hipMalloc(reinterpret_cast<void**>(buf), n * sizeof(T)), "hipMalloc(workspace)");
    if (rc) return rc;
    if (zero) {
        rc = (n * sizeof(T)) % sizeof(int32_t) != 0
                 ? gsp::fail(GSP_E_INVALID_ARG, "zeroed workspaces hold whole 32-bit words")
                 : check_hip(gsp::launch_fill_i32(reinterpret_cast<int32_t*>(*buf),
                                                  (int64_t)(n * sizeof(T) / sizeof(int32_t)), 0, ctx->stream),
                             "fill launch");
        if (rc) return rc;
    }
    *cap = n;
    return GSP_OK;
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
    if (d->block_size > GSP_MAX_BLOCK_SIZE)
        return gsp::fail(GSP_E_UNSUPPORTED, "device pool supports blockSize up to %d (got %d)", GSP_MAX_BLOCK_SIZE,
                         d->block_size);
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
    for (int j = 0; j < gsp_ctx::kSlots && !rc; ++j) {
        rc = check_hip(hipEventCreateWithFlags(&ctx->upload_done[j], hipEventDisableTiming), "hipEventCreate");
        // Recorded once on the idle stream, so the first waits on them pass.
        if (!rc) rc = check_hip(hipEventRecord(ctx->upload_done[j], ctx->own_stream), "hipEventRecord");
    }
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&ctx->aux_done, hipEventDisableTiming), "hipEventCreate");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&ctx->rope_done, hipEventDisableTiming), "hipEventCreate");
    for (int j = 0; j < 2 && !rc; ++j)
        rc = check_hip(hipStreamCreateWithFlags(&ctx->side_stream[j], hipStreamNonBlocking), "hipStreamCreate");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming), "hipEventCreate");
    for (int j = 0; j < 2 && !rc; ++j)
        rc = check_hip(hipEventCreateWithFlags(&ctx->join_ev[j], hipEventDisableTiming), "hipEventCreate");
    // The allocation-free entry point's scratch: look up this device's copy
    // of the array once, with the device current.
    if (!rc) rc = check_hip(gsp::noalloc_setup(device), "hipGetSymbolAddress(scratch)");
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
    for (int j = 0; j < gsp_ctx::kSlots; ++j) {
        if (ctx->staging[j]) (void)hipHostFree(ctx->staging[j]);
        if (ctx->d_step_slot[j]) (void)hipFree(ctx->d_step_slot[j]);
        if (ctx->upload_done[j]) (void)hipEventDestroy(ctx->upload_done[j]);
    }
    if (ctx->aux) (void)hipHostFree(ctx->aux);
    if (ctx->d_aux) (void)hipFree(ctx->d_aux);
    if (ctx->d_mm) (void)hipFree(ctx->d_mm);
    if (ctx->d_mmx) (void)hipFree(ctx->d_mmx);
    if (ctx->d_mmexp) (void)hipFree(ctx->d_mmexp);
    if (ctx->d_mmcnt) (void)hipFree(ctx->d_mmcnt);
    if (ctx->d_mmxs) (void)hipFree(ctx->d_mmxs);
    if (ctx->part) (void)hipFree(ctx->part);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->d_records) (void)hipFree(ctx->d_records);
    if (ctx->aux_done) (void)hipEventDestroy(ctx->aux_done);
    if (ctx->d_rope) (void)hipFree(ctx->d_rope);
    if (ctx->rope_staging) (void)hipHostFree(ctx->rope_staging);
    if (ctx->rope_done) (void)hipEventDestroy(ctx->rope_done);
    for (int j = 0; j < 2; ++j)
        if (ctx->side_stream[j]) (void)hipStreamSynchronize(ctx->side_stream[j]);
    if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
    for (int j = 0; j < 2; ++j) {
        if (ctx->join_ev[j]) (void)hipEventDestroy(ctx->join_ev[j]);
        if (ctx->side_stream[j]) (void)hipStreamDestroy(ctx->side_stream[j]);
    }
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
    if (!rc) rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    for (int j = 0; j < gsp_ctx::kSlots; ++j) ctx->upload_synced[j] = true;
    return GSP_OK;
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

int gsp_set_decode_bins(gsp_ctx* ctx, int32_t bins) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (bins < 0) return gsp::fail(GSP_E_INVALID_ARG, "decode bins must be >= 0 (got %d)", bins);
    ctx->decode_bins_override = bins;
    return GSP_OK;
}

int gsp_set_prefill_path(gsp_ctx* ctx, int32_t path) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (path != GSP_PREFILL_AUTO && path != GSP_PREFILL_TILES && path != GSP_PREFILL_PER_TOKEN)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown prefill path %d", path);
    ctx->prefill_path = path;
    return GSP_OK;
}

int gsp_set_prefill_split(gsp_ctx* ctx, int32_t mode) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (mode != GSP_SPLIT_RECORDS && mode != GSP_SPLIT_IN_TILE)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown prefill split mode %d", mode);
    ctx->prefill_split = mode;
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

}  // extern "C"

namespace {

// Store of n tokens whose block ids and slots are already on the device.
int store_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* d_blocks,
                 const int32_t* d_slots, const float* k_dev, const float* v_dev) {
    const gsp_pool_desc& d = pool->desc;
    gsp::WriteTokensArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.v_block_stride = pool->block_stride_v;
    a.v_layer_offset = (int64_t)layer * pool->layer_stride_v;
    a.v_head_stride = pool->head_stride_v;
    a.block_ids = d_blocks;
    a.slots = d_slots;
    a.k = k_dev;
    a.v = v_dev;
    a.n = n;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    a.v_head_dim = d.v_head_dim;
    return check_hip(gsp::launch_write_tokens(d.kv_dtype == GSP_KV_F16, a, ctx->stream), "write_tokens launch");
}

// The rotation of a RoPE write, checked and resolved for the kernels: the
// angle-rate table on the device (nullptr: freq_base's formula), rope_dim and
// mscale.
struct RopeSetup {
    const double* freq = nullptr;
    double log2_base = 0.0;
    int32_t style = GSP_ROPE_PAIRS;
    int32_t rope_dim = 0;
    float mscale = 1.0f;
};

// Puts the rates `rates` on the device (an entry already holding them, else
// the entry used least recently) and returns its address.
int rope_table(gsp_ctx* ctx, const std::vector<double>& rates, const double** out) {
    int hit = -1, lru = 0;
    for (int e = 0; e < gsp_ctx::kRopeTables; ++e) {
        if (ctx->rope_rates[e] == rates) hit = e;
        if (ctx->rope_used[e] < ctx->rope_used[lru]) lru = e;
    }
    if (hit < 0) {
        bool cap_on = false;
        int rc = is_capturing(ctx->stream, &cap_on);
        if (rc) return rc;
        if (cap_on)
            return gsp::fail(GSP_E_STATE,
                             "a new RoPE table must be copied to the device, which cannot happen while the stream is "
                             "capturing: make one call with this table outside the capture first");
        rc = ensure_device(ctx, &ctx->d_rope, &ctx->d_rope_count,
                           (size_t)gsp_ctx::kRopeTables * gsp::kRopeMaxHalf, false);
        if (!rc) rc = ensure_pinned(&ctx->rope_staging, &ctx->rope_staging_words, 2 * (size_t)gsp::kRopeMaxHalf,
                                    ctx->rope_done, &ctx->rope_pending);
        if (rc) return rc;
        hit = lru;
        double* dst = ctx->d_rope + (size_t)hit * gsp::kRopeMaxHalf;
        std::memcpy(ctx->rope_staging, rates.data(), rates.size() * sizeof(double));
        rc = check_hip(hipMemcpyAsync(dst, ctx->rope_staging, rates.size() * sizeof(double), hipMemcpyHostToDevice,
                                      ctx->stream),
                       "hipMemcpyAsync(rope table)");
        if (!rc) rc = check_hip(hipEventRecord(ctx->rope_done, ctx->stream), "hipEventRecord");
        if (rc) {
            ctx->rope_rates[hit].clear();
            return rc;
        }
        ctx->rope_pending = true;
        ctx->rope_rates[hit] = rates;
    }
    ctx->rope_used[hit] = ++ctx->rope_clock;
    *out = ctx->d_rope + (size_t)hit * gsp::kRopeMaxHalf;
    return GSP_OK;
}

// Checks a rotation against the pool (QuantKernels.RoPE's arguments,
// PagedTransformerRunner.cs:253-264) and resolves it; with `ctx` (after
// set_device) it also places its table on the device.
int check_rope(gsp_ctx* ctx, const gsp_pool* pool, int32_t n_heads, const gsp_rope_spec* spec, const float* q_dev,
               RopeSetup* out) {
    if (!spec) return gsp::fail(GSP_E_INVALID_ARG, "RoPE spec is NULL");
    if (n_heads < 0) return gsp::fail(GSP_E_INVALID_ARG, "nHeads must be >= 0 (got %d)", n_heads);
    if (n_heads > 0 && !q_dev) return gsp::fail(GSP_E_INVALID_ARG, "q is NULL with nHeads %d", n_heads);
    if (spec->style != GSP_ROPE_PAIRS && spec->style != GSP_ROPE_HALVES)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown RoPE pairing %d", spec->style);
    const gsp_pool_desc& d = pool->desc;
    if (d.head_dim % 2 != 0 || d.head_dim > 2 * gsp::kRopeMaxHalf)
        return gsp::fail(GSP_E_UNSUPPORTED, "RoPE needs an even headDim <= %d (got %d)", 2 * gsp::kRopeMaxHalf, d.head_dim);
    const int32_t rope_dim = spec->rope_dim == 0 ? d.head_dim : spec->rope_dim;
    if (rope_dim < 2 || rope_dim > d.head_dim || rope_dim % 2 != 0)
        return gsp::fail(GSP_E_INVALID_ARG, "ropeDim must be even and in [2, headDim %d] (got %d)", d.head_dim,
                         spec->rope_dim);
    const float mscale = spec->mscale == 0.0f ? 1.0f : spec->mscale;
    if (!(mscale > 0.0f) || !std::isfinite(mscale))
        return gsp::fail(GSP_E_INVALID_ARG, "RoPE mscale must be positive and finite");
    if (!spec->inv_freq && (!(spec->freq_base > 0.0f) || !std::isfinite(spec->freq_base)))
        return gsp::fail(GSP_E_INVALID_ARG, "RoPE frequency base must be positive and finite");
    const int32_t half = rope_dim / 2;
    for (int32_t j = 0; spec->inv_freq && j < half; ++j)
        if (!(spec->inv_freq[j] >= 0.0f) || !std::isfinite(spec->inv_freq[j]))
            return gsp::fail(GSP_E_INVALID_ARG, "invFreqTable[%d] must be finite and >= 0", j);
    for (int32_t j = 0; spec->freq_factors && j < half; ++j)
        if (!(spec->freq_factors[j] > 0.0f) || !std::isfinite(spec->freq_factors[j]))
            return gsp::fail(GSP_E_INVALID_ARG, "ropeFreqs[%d] must be positive and finite", j);
    out->style = spec->style;
    out->rope_dim = rope_dim;
    out->mscale = mscale;
    out->freq = nullptr;
    out->log2_base = spec->inv_freq ? 0.0 : std::log2((double)spec->freq_base);
    if (!ctx || (!spec->inv_freq && !spec->freq_factors)) return GSP_OK;
    std::vector<double> rates((size_t)half);
    for (int32_t j = 0; j < half; ++j) {
        double r = spec->inv_freq ? (double)spec->inv_freq[j] : std::exp2(-(2.0 * j / rope_dim) * out->log2_base);
        if (spec->freq_factors) r /= (double)spec->freq_factors[j];
        rates[j] = r;
    }
    return rope_table(ctx, rates, &out->freq);
}

// RoPE then Store of n tokens whose positions, block ids and slots are already on the device.
int rope_store_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* d_pos,
                      const int32_t* d_blocks, const int32_t* d_slots, int32_t n_heads, const RopeSetup& r,
                      float* q_dev, const float* k_dev, const float* v_dev) {
    const gsp_pool_desc& d = pool->desc;
    gsp::RopeWriteArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.v_block_stride = pool->block_stride_v;
    a.v_layer_offset = (int64_t)layer * pool->layer_stride_v;
    a.v_head_stride = pool->head_stride_v;
    a.positions = d_pos;
    a.block_ids = d_blocks;
    a.slots = d_slots;
    a.q = q_dev;
    a.k = k_dev;
    a.v = v_dev;
    a.freq = r.freq;
    a.log2_base = r.log2_base;
    a.n = n;
    a.n_heads = n_heads;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    a.v_head_dim = d.v_head_dim;
    a.style = r.style;
    a.rope_dim = r.rope_dim;
    a.mscale = r.mscale;
    return check_hip(gsp::launch_rope_write(d.kv_dtype == GSP_KV_F16, a, ctx->stream), "rope_write launch");
}

gsp_rope_spec plain_rope(float freq_base, int32_t style) {
    gsp_rope_spec s{};
    s.freq_base = freq_base;
    s.style = style;
    return s;
}

}  // namespace

extern "C" {

int gsp_pool_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* block_ids,
                          const int32_t* slots, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (n < 0) return gsp::fail(GSP_E_INVALID_ARG, "n must be >= 0 (got %d)", n);
    if (n == 0) return GSP_OK;
    if (!block_ids || !slots || !k_dev || !v_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    const gsp_pool_desc& d = pool->desc;
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
    return store_tokens(ctx, pool, layer, n, ctx->d_aux, ctx->d_aux + n, k_dev, v_dev);
}

int gsp_rope_write_tokens_ex(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* positions,
                             const int32_t* block_ids, const int32_t* slots, int32_t n_heads,
                             const gsp_rope_spec* rope, float* q_dev, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (n < 0) return gsp::fail(GSP_E_INVALID_ARG, "n must be >= 0 (got %d)", n);
    if (n == 0) return GSP_OK;
    if (!positions || !block_ids || !slots || !k_dev || !v_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    RopeSetup r;
    int rc = check_rope(nullptr, pool, n_heads, rope, q_dev, &r);
    if (rc) return rc;
    const gsp_pool_desc& d = pool->desc;
    if (layer < 0 || layer >= d.layers) return gsp::fail(GSP_E_INVALID_ARG, "layer %d out of range [0, %d)", layer, d.layers);
    for (int32_t i = 0; i < n; ++i) {
        if (positions[i] < 0) return gsp::fail(GSP_E_INVALID_ARG, "token %d: position %d is negative", i, positions[i]);
        if (block_ids[i] < 0 || block_ids[i] >= d.total_blocks)
            return gsp::fail(GSP_E_INVALID_ARG, "block id %d out of range [0, %d)", block_ids[i], d.total_blocks);
        if (slots[i] < 0 || slots[i] >= d.block_size)
            return gsp::fail(GSP_E_INVALID_ARG, "slot %d out of range [0, %d)", slots[i], d.block_size);
    }
    rc = set_device(ctx);
    if (!rc) rc = check_rope(ctx, pool, n_heads, rope, q_dev, &r);
    if (rc) return rc;
    const size_t words = 3 * (size_t)n;
    rc = ensure_pinned(&ctx->aux, &ctx->aux_words, words, ctx->aux_done, &ctx->aux_pending);
    if (!rc) rc = ensure_device(ctx, &ctx->d_aux, &ctx->d_aux_words, words, false);
    if (rc) return rc;
    std::memcpy(ctx->aux, positions, n * sizeof(int32_t));
    std::memcpy(ctx->aux + n, block_ids, n * sizeof(int32_t));
    std::memcpy(ctx->aux + 2 * (size_t)n, slots, n * sizeof(int32_t));
    rc = check_hip(hipMemcpyAsync(ctx->d_aux, ctx->aux, words * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream),
                   "hipMemcpyAsync(rope ids)");
    if (!rc) rc = check_hip(hipEventRecord(ctx->aux_done, ctx->stream), "hipEventRecord");
    if (rc) return rc;
    ctx->aux_pending = true;
    return rope_store_tokens(ctx, pool, layer, n, ctx->d_aux, ctx->d_aux + n, ctx->d_aux + 2 * (size_t)n, n_heads, r,
                             q_dev, k_dev, v_dev);
}

int gsp_rope_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* positions,
                          const int32_t* block_ids, const int32_t* slots, int32_t n_heads, float freq_base,
                          int32_t style, float* q_dev, const float* k_dev, const float* v_dev) {
    const gsp_rope_spec spec = plain_rope(freq_base, style);
    return gsp_rope_write_tokens_ex(ctx, pool, layer, n, positions, block_ids, slots, n_heads, &spec, q_dev, k_dev,
                                    v_dev);
}

}  // extern "C"

namespace {

// The packed step's own K/V write: query token i's K and V go to the slot of
// its position (positions[b] + i of its row), read from the device copy of
// the step, so every layer of a tick reuses one upload.
int check_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, const float* k_dev, const float* v_dev) {
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (!ctx->step_valid) return gsp::fail(GSP_E_STATE, "gsp_step_pack must succeed before a step write");
    const gsp_pool_desc& d = pool->desc;
    if (d.heads_kv != ctx->step_heads_kv || d.total_blocks < ctx->step_blocks || d.block_size != ctx->step_block_size)
        return gsp::fail(GSP_E_INVALID_ARG,
                         "the step was packed for a pool with %d KV heads, %d blocks and %d-token pages",
                         ctx->step_heads_kv, ctx->step_blocks, ctx->step_block_size);
    if (ctx->max_id >= d.total_blocks)
        return gsp::fail(GSP_E_INVALID_ARG, "block id %d out of range [0, %d)", ctx->max_id, d.total_blocks);
    if (layer < 0 || layer >= d.layers) return gsp::fail(GSP_E_INVALID_ARG, "layer %d out of range [0, %d)", layer, d.layers);
    if (ctx->info.total_q > 0 && (!k_dev || !v_dev)) return gsp::fail(GSP_E_INVALID_ARG, "k/v must not be NULL");
    return set_device(ctx);
}

}  // namespace

extern "C" {

int gsp_pool_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    int rc = check_write_step(ctx, pool, layer, k_dev, v_dev);
    if (rc) return rc;
    const int32_t n = ctx->info.total_q;
    if (n == 0) return GSP_OK;
    bool cap = false;
    rc = step_begin(ctx, &cap);
    if (rc) return rc;
    const int32_t* wr = ctx->d_step + ctx->off_wr;
    rc = store_tokens(ctx, pool, layer, n, wr + n, wr + 2 * (size_t)n, k_dev, v_dev);
    const int rd = step_done(ctx, cap);
    return rc ? rc : rd;
}

int gsp_rope_write_step_ex(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n_heads, const gsp_rope_spec* rope,
                           float* q_dev, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    int rc = check_write_step(ctx, pool, layer, k_dev, v_dev);
    if (rc) return rc;
    RopeSetup r;
    rc = check_rope(nullptr, pool, n_heads, rope, q_dev, &r);
    if (rc) return rc;
    const int32_t n = ctx->info.total_q;
    if (n == 0) return GSP_OK;
    bool cap = false;
    rc = step_begin(ctx, &cap);
    if (!rc) rc = check_rope(ctx, pool, n_heads, rope, q_dev, &r);
    if (rc) return rc;
    const int32_t* wr = ctx->d_step + ctx->off_wr;
    rc = rope_store_tokens(ctx, pool, layer, n, wr, wr + n, wr + 2 * (size_t)n, n_heads, r, q_dev, k_dev, v_dev);
    const int rd = step_done(ctx, cap);
    return rc ? rc : rd;
}

int gsp_rope_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n_heads, float freq_base, int32_t style,
                        float* q_dev, const float* k_dev, const float* v_dev) {
    const gsp_rope_spec spec = plain_rope(freq_base, style);
    return gsp_rope_write_step_ex(ctx, pool, layer, n_heads, &spec, q_dev, k_dev, v_dev);
}

// Q8_0 and K-quant products with at least this many outputs (batch x out_dim)
// take the fp16 path (unless the small-batch form takes them): for Q8_0
// measured faster from Qwen2.5-7B's 3584 x 3584 projection at 64 rows
// (229376 outputs: 27.8 vs 31.2 us) upwards, slower for 8192 x 8192 at 16 rows
// (131072 outputs: 57.5 vs 51 us) and 3584 x 512 at 64 rows (21.5 vs 16.2 us).
constexpr int64_t kMatmulF16MinOutputs = 196608;
// Q8_0 and K-quant products of at most 64 batch rows with at least this many
// outputs take the small-batch fp16 form: for Q8_0 measured faster than the
// other two forms from 8192 x 8192 at 16 rows (131072 outputs: 40.6 vs 43.7 us)
// and Qwen2.5-7B's 3584 x 3584 at 64 rows (22.1 vs 24.3 us), slower for
// 896 x 896 at 8 rows (7168 outputs: 15.8 vs 6.9 us), whose product is too
// small to fill the chip.  Between 16384 and 65536 outputs it was faster
// than the fp32 form on most shapes measured (4096 x 1024 at 32 rows: Q8_0
// 18.3 -> 14.8 us, Q6_K 19.6 -> 15.5 us; 8192 x 1024 at 16 rows: Q6_K 23.4
// -> 18.2 us) and at most 0.5 us slower on the others (3584 x 512 at 64 rows:
// Q4_K 17.0 -> 17.25 us, Q6_K 18.6 -> 19.1 us, while Q8_0 gains 16.8 -> 15.8).
constexpr int64_t kMatmulSmallMinOutputs = 16384;

int gsp_matmul_batch(gsp_ctx* ctx, int32_t w_type, const void* w_dev, const float* x_dev, float* y_dev,
                     int32_t in_dim, int32_t out_dim, int32_t batch) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (in_dim < 0 || out_dim < 0 || batch < 0)
        return gsp::fail(GSP_E_INVALID_ARG, "negative size (inDim %d, outDim %d, batch %d)", in_dim, out_dim, batch);
    if (batch == 0 || out_dim == 0) return GSP_OK;
    if (!w_dev || !x_dev || !y_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    if (w_type != GSP_WTYPE_F32 && w_type != GSP_WTYPE_Q8_0 && w_type != GSP_WTYPE_Q4_K && w_type != GSP_WTYPE_Q6_K)
        return gsp::fail(GSP_E_UNSUPPORTED,
                         "weight type %d: only F32 (%d), Q8_0 (%d), Q4_K (%d) and Q6_K (%d) are supported", w_type,
                         GSP_WTYPE_F32, GSP_WTYPE_Q8_0, GSP_WTYPE_Q4_K, GSP_WTYPE_Q6_K);
    const bool kquant = w_type == GSP_WTYPE_Q4_K || w_type == GSP_WTYPE_Q6_K;
    if (in_dim == 0 || in_dim % (kquant ? 256 : 64) != 0)
        return gsp::fail(GSP_E_UNSUPPORTED, "inDim must be a positive multiple of %d for weight type %d (got %d)",
                         kquant ? 256 : 64, w_type, in_dim);
    const uintptr_t walign = w_type == GSP_WTYPE_F32 ? 16 : w_type == GSP_WTYPE_Q6_K ? 2 : 4;
    if (reinterpret_cast<uintptr_t>(w_dev) % walign != 0 || reinterpret_cast<uintptr_t>(x_dev) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(y_dev) % 4 != 0)
        return gsp::fail(GSP_E_INVALID_ARG, "weights must be %d-byte aligned, x 16-byte aligned, y 4-byte aligned",
                         (int)walign);
    int rc = set_device(ctx);
    if (rc) return rc;
    if ((w_type == GSP_WTYPE_Q8_0 || w_type == GSP_WTYPE_Q4_K || w_type == GSP_WTYPE_Q6_K) && batch <= 64 &&
        (int64_t)batch * out_dim >= kMatmulSmallMinOutputs &&
        (in_dim / 64 + gsp::matmul_small_range_chunks_max() - 1) / gsp::matmul_small_range_chunks_max() <=
            gsp::matmul_small_max_splits(batch)) {
        // Small batches: about two workgroups (64 weight rows, every batch row)
        // per CU and no more K ranges than the merge holds.  Ranges whose
        // weights fit the workgroup's LDS when the merge allows enough of them;
        // else longer ranges, which the workgroup walks in passes.  The partial
        // offsets are 32-bit.
        const int64_t chunks = in_dim / 64;
        const int64_t tiles = (out_dim + 63) / 64;
        const int64_t maxs = gsp::matmul_small_max_splits(batch);
        const int64_t lo = (chunks + gsp::matmul_small_chunks(batch) - 1) / gsp::matmul_small_chunks(batch);
        // Rounded down, so the grid fits the slots in one round: rounded up it
        // spilled a few workgroups into a second round (3584 x 3584 at 32 rows:
        // 560 workgroups, Q8_0 19.9 us, against 448 and 16.9 us).
        const int64_t want = std::max<int64_t>(1, 2 * (int64_t)std::max(1, ctx->num_cus) / tiles);
        int64_t splits = lo <= maxs ? std::max(lo, std::min({want, maxs, chunks}))
                                    : std::max<int64_t>((chunks + gsp::matmul_small_range_chunks_max() - 1) /
                                                            gsp::matmul_small_range_chunks_max(),
                                                        std::min(want, maxs));
        // Outputs that fill the CU slots (two per CU) at least twice over (an
        // LM head) need no K split: one range per tile, walked in passes, with
        // no partials and no merge.  Measured faster from 1024 tiles up (on 256
        // CUs: 3584 x 65536 at 64 rows 150 -> 118 us for Q8_0, 160 -> 125 us
        // for Q4_K; Llama-3's 4096 x 128256 head at 8 rows 208 -> 185 us for
        // Q8_0); from 512 tiles up it lost where a second round of workgroups
        // stays nearly empty (4096 x 40960 at 32 rows 83 -> 97 us for Q8_0).
        if (tiles >= 4 * (int64_t)std::max(1, ctx->num_cus) && chunks <= gsp::matmul_small_range_chunks_max())
            splits = 1;
        int64_t per = (chunks + splits - 1) / splits;
        if (w_type == GSP_WTYPE_Q6_K) per += per & 1;  // Q6_K ranges start on a 128-weight half of a super-block
        splits = (chunks + per - 1) / per;
        gsp::MatmulArgs a{};
        a.w = w_dev;
        a.x = x_dev;
        a.y = y_dev;
        a.w_type = w_type;
        a.in_dim = in_dim;
        a.out_dim = out_dim;
        a.batch = batch;
        a.splits = (int32_t)splits;
        a.chunks_per_split = (int32_t)per;
        rc = ensure_device(ctx, &ctx->d_mmx, &ctx->d_mmx_halves, (size_t)gsp::matmul_small_x_halves(batch, in_dim), false);
        if (!rc) rc = ensure_device(ctx, &ctx->d_mmexp, &ctx->d_mmexp_words, (size_t)splits * batch, false);
        if (!rc && splits > 1) rc = ensure_device(ctx, &ctx->d_mm, &ctx->d_mm_floats, (size_t)splits * batch * tiles * 64, false);
        if (!rc && splits > 1) rc = ensure_device(ctx, &ctx->d_mmcnt, &ctx->d_mmcnt_words, (size_t)tiles, true);
        if (!rc && w_type == GSP_WTYPE_Q4_K)
            rc = ensure_device(ctx, &ctx->d_mmxs, &ctx->d_mmxs_floats, (size_t)splits * 2 * per * 64, false);
        if (rc) return rc;
        a.xh = ctx->d_mmx;  // x in tile order, both halves
        a.xl = ctx->d_mmx;
        a.xexp = ctx->d_mmexp;
        a.split_out = splits > 1 ? ctx->d_mm : nullptr;
        a.counters = splits > 1 ? ctx->d_mmcnt : nullptr;
        a.xsum = w_type == GSP_WTYPE_Q4_K ? ctx->d_mmxs : nullptr;
        return check_hip(gsp::launch_matmul_small(a, ctx->stream), "matmul launch");
    }
    // Split K over grid.z until the grid has about two workgroups (64 weight rows
    // x 64 batch rows each) per CU, keeping at least two 64-wide chunks in every
    // range so that loads overlap the products.
    const int64_t chunks = in_dim / 64;
    const int64_t base = (int64_t)((out_dim + 63) / 64) * ((batch + 63) / 64);
    const int64_t want = std::max<int64_t>(1, (2 * (int64_t)std::max(1, ctx->num_cus) + base - 1) / base);
    const int64_t splits_max = std::max<int64_t>(1, chunks / 2);
    int64_t splits = std::min(want, splits_max);
    const int64_t per = (chunks + splits - 1) / splits;
    splits = (chunks + per - 1) / per;
    gsp::MatmulArgs a{};
    a.w = w_dev;
    a.x = x_dev;
    a.y = y_dev;
    a.split_out = nullptr;
    a.w_type = w_type;
    a.in_dim = in_dim;
    a.out_dim = out_dim;
    a.batch = batch;
    a.splits = (int32_t)splits;
    a.chunks_per_split = (int32_t)per;
    a.xh = nullptr;
    a.xl = nullptr;
    a.xexp = nullptr;
    if ((w_type == GSP_WTYPE_Q8_0 || w_type == GSP_WTYPE_Q4_K || w_type == GSP_WTYPE_Q6_K) &&
        (int64_t)batch * out_dim >= kMatmulF16MinOutputs) {
        // Large Q8_0 and K-quant products run on the fp16 matrix cores with x as
        // scaled fp16 pairs (Q4_K also with x's block sums for its min term);
        // below the threshold the pre-pass launch costs more than it saves.
        const size_t halves = (size_t)batch * in_dim;
        rc = ensure_device(ctx, &ctx->d_mmx, &ctx->d_mmx_halves, 2 * halves, false);
        if (!rc) rc = ensure_device(ctx, &ctx->d_mmexp, &ctx->d_mmexp_words, (size_t)batch, false);
        if (!rc && w_type == GSP_WTYPE_Q4_K)
            rc = ensure_device(ctx, &ctx->d_mmxs, &ctx->d_mmxs_floats, (size_t)batch * (in_dim / 32), false);
        if (rc) return rc;
        a.xh = ctx->d_mmx;
        a.xl = ctx->d_mmx + halves;
        a.xexp = ctx->d_mmexp;
        a.xsum = w_type == GSP_WTYPE_Q4_K ? ctx->d_mmxs : nullptr;
    }
    if (splits > 1) {
        rc = ensure_device(ctx, &ctx->d_mm, &ctx->d_mm_floats, (size_t)splits * batch * out_dim, false);
        if (rc) return rc;
        a.split_out = ctx->d_mm;
    }
    return check_hip(gsp::launch_matmul(a, ctx->stream), "matmul launch");
}

int gsp_block_allocator_attach_pool(gsp_block_allocator* a, gsp_ctx* ctx, gsp_pool* pool) {
    gsp::clear_error();
    if (!a) return gsp::fail(GSP_E_INVALID_ARG, "allocator is NULL");
    if ((ctx == nullptr) != (pool == nullptr)) return gsp::fail(GSP_E_INVALID_ARG, "ctx and pool must both be set or both NULL");
    if (pool && pool->desc.total_blocks < a->total)
        return gsp::fail(GSP_E_INVALID_ARG, "the pool holds %d blocks, the allocator %d", pool->desc.total_blocks,
                         a->total);
    a->ctx = ctx;
    a->pool = pool;
    a->copy_page = pool ? gsp_pool_copy_block : nullptr;
    return GSP_OK;
}

int gsp_pool_copy_block(gsp_ctx* ctx, gsp_pool* pool, int32_t src, int32_t dst, int32_t valid_tokens) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    const gsp_pool_desc& d = pool->desc;
    if (src < 0 || src >= d.total_blocks || dst < 0 || dst >= d.total_blocks)
        return gsp::fail(GSP_E_INVALID_ARG, "block ids (%d, %d) out of range [0, %d)", src, dst, d.total_blocks);
    if (valid_tokens <= 0) return GSP_OK;
    int rc = set_device(ctx);
    if (rc) return rc;
    gsp::CopyBlockArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.block_stride = pool->block_stride_k;
    a.head_stride = pool->head_stride_k;
    a.v_block_stride = pool->block_stride_v;
    a.v_head_stride = pool->head_stride_v;
    a.src = src;
    a.dst = dst;
    a.valid_tokens = std::min(valid_tokens, d.block_size);
    a.layers = d.layers;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    a.v_head_dim = d.v_head_dim;
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

int gsp_step_pack(gsp_ctx* ctx, const gsp_pool* pool, const gsp_step_desc* desc) {
    gsp::clear_error();
    if (!ctx || !pool || !desc) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool/desc is NULL");
    const auto t_pack0 = std::chrono::steady_clock::now();
    {
        // Refused before anything changes: the step already packed stays valid.
        bool cap_on = false;
        const int rc = is_capturing(ctx->stream, &cap_on);
        if (rc) return rc;
        if (cap_on)
            return gsp::fail(GSP_E_STATE,
                             "gsp_step_pack cannot run while the stream is capturing: it stages the step in "
                             "host memory; pack eagerly, then capture gsp_attention_step");
    }
    ctx->step_valid = false;
    const gsp_pool_desc& pd = pool->desc;
    gsp::PlanPool pp;
    pp.total_blocks = pd.total_blocks;
    pp.layers = pd.layers;
    pp.heads_kv = pd.heads_kv;
    pp.head_dim = pd.head_dim;
    pp.v_head_dim = pd.v_head_dim;
    pp.block_size = pd.block_size;
    pp.kv_dtype = pd.kv_dtype;
    gsp::PlanOptions po;
    po.num_cus = ctx->num_cus;
    po.split_pages_override = ctx->split_pages_override;
    po.decode_bins_override = ctx->decode_bins_override;
    po.prefill_path = ctx->prefill_path;
    po.prefill_split = ctx->prefill_split;
    gsp::StepPlan& plan = ctx->plan;
    int rc = ctx->planner.plan(pp, desc, po, plan);
    if (rc) return rc;
    const int32_t H = pd.heads_kv;
    const size_t words = plan.image.size();
    const size_t words16 = align_up(words, 4);  // the upload moves 16-byte words

    rc = set_device(ctx);
    if (rc) return rc;
    // The other slot than the step packed last: its kernels may still run.
    const int slot = ctx->slot ^ 1;
    const auto t_wait0 = std::chrono::steady_clock::now();
    if (ctx->slot_captured[slot]) {  // replays of a graph that read this slot
        rc = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (rc) return rc;
        ctx->slot_captured[slot] = false;
    }
    {
        const size_t had = ctx->staging_words[slot];  // changes when the buffer is replaced
        rc = ensure_pinned(&ctx->staging[slot], &ctx->staging_words[slot], words16, ctx->upload_done[slot],
                           &ctx->upload_pending[slot], hipHostMallocMapped | hipHostMallocCoherent);
        ctx->info.pack_wait_ns =
            std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t_wait0).count();
        if (!rc && (ctx->staging_words[slot] != had || !ctx->staging_dev[slot])) {
            void* dp = nullptr;
            rc = check_hip(hipHostGetDevicePointer(&dp, ctx->staging[slot], 0), "hipHostGetDevicePointer(staging)");
            ctx->staging_dev[slot] = rc ? nullptr : dp;
        }
    }
    if (!rc) rc = ensure_device(ctx, &ctx->d_step_slot[slot], &ctx->d_step_words[slot], words16, false);
    // The split workspace for any group up to the decode tile, so that a
    // captured gsp_attention_step of this step never has to grow it.
    if (!rc && plan.num_slots > 0)
        rc = ensure_device(ctx, &ctx->part, &ctx->part_floats,
                           (size_t)plan.num_slots * gsp::kMaxGroupMfma * (size_t)(pd.v_head_dim + 2), false);
    if (!rc && plan.num_slots > 0)
        rc = ensure_device(ctx, &ctx->counters, &ctx->counter_words, (size_t)plan.total_q * H, true);
    // The split records, so that a captured gsp_attention_step never grows them.
    if (!rc && plan.num_records > 0)
        rc = ensure_device(ctx, &ctx->d_records, &ctx->d_records_bytes,
                           (size_t)plan.num_records * (size_t)gsp::prefill_record_bytes(pd.head_dim), false);
    if (rc) return rc;

    // One copy for the whole step, on the context's stream (behind the
    // kernels that read this slot's previous step), then the event that frees
    // the pinned buffer.  The pad words up to a 16-byte word are zeroed.
    std::memcpy(ctx->staging[slot], plan.image.data(), words * sizeof(int32_t));
    for (size_t j = words; j < words16; ++j) ctx->staging[slot][j] = 0;
    rc = check_hip(gsp::launch_upload_step(ctx->staging_dev[slot], ctx->d_step_slot[slot], (int64_t)(words16 / 4),
                                           ctx->stream),
                   "step upload launch");
    if (!rc) rc = check_hip(hipEventRecord(ctx->upload_done[slot], ctx->stream), "hipEventRecord");
    if (rc) return rc;
    ctx->upload_pending[slot] = true;
    ctx->upload_synced[slot] = false;
    ctx->slot = slot;
    ctx->d_step = ctx->d_step_slot[slot];

    ctx->off_rows = plan.off_rows;
    ctx->off_ids = plan.off_ids;
    ctx->off_ctx = plan.off_ctx;
    ctx->off_wr = plan.off_wr;
    ctx->off_units = plan.off_units;
    ctx->off_tiles = plan.off_tiles;
    ctx->off_split = plan.off_split;
    ctx->off_bins = plan.off_bins;
    ctx->num_split_items = plan.num_split_items;
    ctx->split_max_pairs = plan.split_max_pairs;
    ctx->num_records = plan.num_records;
    ctx->records_head_dim = plan.num_records > 0 ? pd.head_dim : 0;
    ctx->num_bins = plan.num_bins;
    ctx->max_id = plan.max_id;
    ctx->num_slots = (int32_t)plan.num_slots;
    ctx->num_units = plan.num_units;
    ctx->num_tiles = plan.num_tiles;
    ctx->step_heads_kv = H;
    ctx->step_blocks = pd.total_blocks;
    ctx->step_block_size = pd.block_size;
    ctx->step_page_tokens = plan.page_tokens;
    ctx->step_tile_pages = plan.tile_pages;
    ctx->step_tileable = plan.tileable;
    ctx->info.num_rows = plan.num_rows;
    ctx->info.total_q = (int32_t)plan.total_q;
    ctx->info.packed_pages = (int32_t)plan.packed_pages;
    ctx->info.heads_kv = H;
    ctx->info.decode_units = plan.num_units;
    ctx->info.split_pairs = (int32_t)plan.pairs_split;
    ctx->info.partial_slots = (int32_t)plan.num_slots;
    ctx->info.pages_per_split = plan.target;
    ctx->info.kv_tokens = plan.kv_tokens;
    ctx->info.staging_bytes = (int64_t)(words * sizeof(int32_t));
    ctx->info.prefill_tiles = plan.num_tiles;
    ctx->info.prefill_queries = (int32_t)plan.tiled_queries;
    ctx->info.prefill_pairs = plan.tiled_pairs;
    ctx->info.decode_bins = plan.num_bins;
    ctx->info.split_records = (int32_t)plan.num_records;
    ctx->info.pack_host_ns =
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t_pack0).count();
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
    if (!rc) rc = check_hip(hipEventSynchronize(ctx->upload_done[ctx->slot]), "hipEventSynchronize(upload)");
    if (rc) return rc;
    ctx->upload_synced[ctx->slot] = true;
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

}  // extern "C"

namespace {

// Split-KV workspace of one attention launch: the context's own (grown on
// demand, outside graph capture) or a fixed device array (the allocation-free
// entry point), whose counters are cleared before every launch.
struct Workspace {
    float* part = nullptr;
    size_t part_floats = 0;
    int32_t* counters = nullptr;
    size_t counter_words = 0;
};

int attention_launch(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads, const float* q_dev,
                     float* out_dev, float attn_scale, const float* sink_logit, const Workspace* fixed) {
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (!ctx->step_valid) return gsp::fail(GSP_E_STATE, "gsp_step_pack must succeed before gsp_attention_step");
    const gsp_pool_desc& d = pool->desc;
    if (sink_logit) return gsp::fail(GSP_E_UNSUPPORTED, "attention sinks are not supported on the GPU path");
    // The reference GPU runner's bound (CudaPagedTransformerRunner.cs:408-412);
    // odd widths as in the CPU kernel's generic path (PagedAttentionKernel.cs:326-370).
    if (d.head_dim > 256 || d.v_head_dim > 256)
        return gsp::fail(GSP_E_UNSUPPORTED, "headDim (%d) and vHeadDim (%d) must be at most 256", d.head_dim,
                         d.v_head_dim);
    if (layer < 0 || layer >= d.layers) return gsp::fail(GSP_E_INVALID_ARG, "layer %d out of range [0, %d)", layer, d.layers);
    if (n_heads < 1 || n_heads % d.heads_kv != 0)
        return gsp::fail(GSP_E_INVALID_ARG, "nHeads (%d) must be a positive multiple of nHeadsKv (%d)", n_heads, d.heads_kv);
    if (d.heads_kv != ctx->step_heads_kv || d.total_blocks < ctx->step_blocks || d.block_size != ctx->step_block_size ||
        (ctx->num_tiles > 0 && !ctx->step_tileable))
        return gsp::fail(GSP_E_INVALID_ARG,
                         "the step was packed for a pool with %d KV heads, %d blocks and %d-token pages",
                         ctx->step_heads_kv, ctx->step_blocks, ctx->step_block_size);
    const int group = n_heads / d.heads_kv;
    // The matrix-core kernel serves any group, 16 query heads per tile; the
    // DPP kernel is kept for explicit selection (fixed shapes, groups up to 8).
    const bool use_mfma = ctx->decode_path != GSP_DECODE_DPP;
    if (!use_mfma && ctx->num_units > 0 &&
        (group > gsp::kMaxGroup || d.head_dim != d.v_head_dim || (d.head_dim != 64 && d.head_dim != 128) ||
         ctx->step_page_tokens != gsp::kBlockSize))
        return gsp::fail(GSP_E_UNSUPPORTED,
                         "the DPP decode kernel serves headDim 64 or 128, 16-token pages and groups up to %d",
                         gsp::kMaxGroup);
    const int tiles = use_mfma ? (group + gsp::kDecodeTileHeads - 1) / gsp::kDecodeTileHeads : 1;
    const int slot_heads = use_mfma ? std::min(group, gsp::kDecodeTileHeads) : group;
    if (ctx->max_id >= d.total_blocks)
        return gsp::fail(GSP_E_INVALID_ARG, "block id %d out of range [0, %d)", ctx->max_id, d.total_blocks);
    if (ctx->num_units == 0 && ctx->num_tiles == 0) return GSP_OK;
    if (!q_dev || !out_dev) return gsp::fail(GSP_E_INVALID_ARG, "q/out must not be NULL");
    int rc = set_device(ctx);
    if (rc) return rc;

    const int32_t slots = ctx->num_slots;
    float* part = ctx->part;
    int32_t* counters = ctx->counters;
    const size_t counter_need = (size_t)ctx->info.total_q * d.heads_kv * tiles;
    if (slots > 0) {
        const size_t part_need = (size_t)slots * tiles * slot_heads * (d.v_head_dim + 2);
        if (fixed) {
            if (part_need > fixed->part_floats || counter_need > fixed->counter_words)
                return gsp::fail(GSP_E_INVALID_ARG,
                                 "the step needs %zu bytes of split-KV partials and %zu counters; the "
                                 "allocation-free entry point holds %zu bytes and %zu counters",
                                 part_need * sizeof(float), counter_need, fixed->part_floats * sizeof(float),
                                 fixed->counter_words);
            part = fixed->part;
            counters = fixed->counters;
        } else {
            rc = ensure_device(ctx, &ctx->part, &ctx->part_floats, part_need, false);
            // Counters start at zero and every launch leaves them at zero.
            if (!rc) rc = ensure_device(ctx, &ctx->counters, &ctx->counter_words, counter_need, true);
            if (rc) return rc;
            part = ctx->part;
            counters = ctx->counters;
        }
    }

    bool capturing = false;
    rc = step_begin(ctx, &capturing);
    if (rc) return rc;
    if (fixed && slots > 0) {
        // The array keeps whatever the last call on this GPU left: clear the
        // counters this launch uses (every launch leaves its own at zero).
        rc = check_hip(gsp::launch_fill_i32(counters, (int64_t)counter_need, 0, ctx->stream), "fill launch");
        if (rc) return rc;
    }

    gsp::DecodeArgs a;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    // Pool pages above 16 tokens are read as kernel pages of step_page_tokens
    // tokens whose ids count in kernel page strides (gsp_step_plan.h).
    const bool kernel_pages = ctx->step_page_tokens != d.block_size;
    a.block_stride = kernel_pages ? (int64_t)ctx->step_page_tokens * d.head_dim : pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.v_block_stride = kernel_pages ? (int64_t)ctx->step_page_tokens * d.v_head_dim : pool->block_stride_v;
    a.v_layer_offset = (int64_t)layer * pool->layer_stride_v;
    a.v_head_stride = pool->head_stride_v;
    a.units = reinterpret_cast<const DecodeUnit*>(ctx->d_step + ctx->off_units);
    a.bin_rest = ctx->d_step + ctx->off_bins;
    a.bt_ids = ctx->d_step + ctx->off_ids;
    a.q = q_dev;
    a.out = out_dev;
    a.part_o = slots > 0 ? part : nullptr;
    a.part_ml = slots > 0 ? part + (size_t)slots * tiles * slot_heads * d.v_head_dim : nullptr;
    a.counters = slots > 0 ? counters : nullptr;
    a.n_heads = n_heads;
    a.n_kv = d.heads_kv;
    a.group = group;
    a.scale_log2 = attn_scale * 1.4426950408889634f;
    a.head_dim = d.head_dim;
    a.v_head_dim = d.v_head_dim;
    a.block_size = ctx->step_page_tokens;
    a.tile_pages = ctx->step_tile_pages;
    a.total_q = ctx->info.total_q;
    a.num_slots = slots;
    a.slot_heads = slot_heads;
    const int f16 = d.kv_dtype == GSP_KV_F16;
    gsp::PrefillArgs p;
    p.k_pool = a.k_pool;
    p.v_pool = a.v_pool;
    p.block_stride = a.block_stride;
    p.layer_offset = a.layer_offset;
    p.head_stride = a.head_stride;
    p.tiles = reinterpret_cast<const PrefillTile*>(ctx->d_step + ctx->off_tiles);
    p.bt_ids = a.bt_ids;
    p.q = q_dev;
    p.out = out_dev;
    p.n_heads = n_heads;
    p.n_kv = d.heads_kv;
    p.group = group;
    p.scale_log2 = a.scale_log2;
    p.records = nullptr;
    // fp32 tiles read the step's split records, written here for this layer
    // just before the tiles on the tiles' stream (the allocation-free entry
    // point has no room for them: its tiles split their own pages).
    const bool use_records = !fixed && ctx->num_tiles > 0 && ctx->num_records > 0 && !f16 &&
                             ctx->records_head_dim == d.head_dim &&
                             ctx->d_records_bytes >= (size_t)ctx->num_records * (size_t)gsp::prefill_record_bytes(d.head_dim);
    auto launch_split = [&](hipStream_t s) -> int {
        if (!use_records) return GSP_OK;
        gsp::PrefillSplitArgs sa;
        sa.k_pool = p.k_pool;
        sa.v_pool = p.v_pool;
        sa.block_stride = p.block_stride;
        sa.layer_offset = p.layer_offset;
        sa.head_stride = p.head_stride;
        sa.items = reinterpret_cast<const gsp::PrefillSplitItem*>(ctx->d_step + ctx->off_split);
        sa.bt_ids = p.bt_ids;
        sa.records = ctx->d_records;
        p.records = ctx->d_records;
        return check_hip(gsp::launch_prefill_split(d.head_dim, ctx->num_split_items, ctx->split_max_pairs, sa, s),
                         "prefill split launch");
    };
    // Decode units stream from HBM and prefill tiles keep the matrix cores
    // busy.  With both in the step and the matrix-core decode (tiles exist
    // only for its fixed shapes), one kernel runs both kinds of workgroup side
    // by side.  With the DPP decode, each kernel goes to its own side stream,
    // forked here and joined back below.
    if (use_mfma && ctx->num_units > 0 && ctx->num_tiles > 0) {
        rc = launch_split(ctx->stream);
        if (!rc)
            rc = check_hip(gsp::launch_mixed_mfma(d.head_dim, f16, ctx->num_bins, ctx->num_tiles, a, p, ctx->stream),
                           "mixed step launch");
        const int rd = step_done(ctx, capturing);
        return rc ? rc : rd;
    }
    const bool fork = ctx->num_units > 0 && ctx->num_tiles > 0;
    hipStream_t decode_stream = fork ? ctx->side_stream[0] : ctx->stream;
    hipStream_t tile_stream = fork ? ctx->side_stream[1] : ctx->stream;
    if (fork) {
        rc = check_hip(hipEventRecord(ctx->fork_ev, ctx->stream), "hipEventRecord(fork)");
        for (int j = 0; j < 2 && !rc; ++j)
            rc = check_hip(hipStreamWaitEvent(ctx->side_stream[j], ctx->fork_ev, 0), "hipStreamWaitEvent(fork)");
        if (rc) return rc;
    }
    if (ctx->num_units > 0) {
        rc = use_mfma ? check_hip(gsp::launch_decode_mfma(f16, ctx->num_bins, a, decode_stream), "decode (mfma) launch")
                      : check_hip(gsp::launch_decode(d.head_dim, f16, ctx->num_bins, a, decode_stream),
                                  "decode (dpp) launch");
        if (rc && fork) {
            // Join what was forked, so the side streams hold nothing of this step.
            for (int j = 0; j < 2; ++j)
                if (hipEventRecord(ctx->join_ev[j], ctx->side_stream[j]) == hipSuccess)
                    (void)hipStreamWaitEvent(ctx->stream, ctx->join_ev[j], 0);
        }
        if (rc) return rc;
    }
    if (ctx->num_tiles > 0) {
        rc = launch_split(tile_stream);
        if (!rc)
            rc = check_hip(gsp::launch_prefill_mfma(d.head_dim, f16, ctx->num_tiles, p, tile_stream), "prefill launch");
    }
    if (fork) {
        for (int j = 0; j < 2; ++j) {
            const int jc = check_hip(hipEventRecord(ctx->join_ev[j], ctx->side_stream[j]), "hipEventRecord(join)");
            const int jw =
                jc ? jc : check_hip(hipStreamWaitEvent(ctx->stream, ctx->join_ev[j], 0), "hipStreamWaitEvent(join)");
            if (!rc) rc = jw;
        }
    }
    const int rd = step_done(ctx, capturing);
    return rc ? rc : rd;
}

// Layout of the fixed scratch: counters first, then the partials.
constexpr size_t kNoallocCounterWords = GSP_NOALLOC_COUNTERS;
static_assert(kNoallocCounterWords * sizeof(int32_t) < GSP_NOALLOC_SCRATCH_BYTES, "counters fit the scratch");

}  // namespace

extern "C" {

int gsp_attention_step(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads, const float* q_dev,
                       float* out_dev, float attn_scale, const float* sink_logit) {
    gsp::clear_error();
    return attention_launch(ctx, pool, layer, n_heads, q_dev, out_dev, attn_scale, sink_logit, nullptr);
}

int gsp_attention_step_noalloc(gsp_ctx* ctx, const gsp_pool* pool, int32_t layer, int32_t n_heads,
                               const float* q_dev, float* out_dev, float attn_scale, const float* sink_logit) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    char* base = static_cast<char*>(gsp::noalloc_scratch(ctx->device));
    if (!base) return gsp::fail(GSP_E_STATE, "the scratch array of device %d was not set up", ctx->device);
    Workspace ws;
    ws.counters = reinterpret_cast<int32_t*>(base);
    ws.counter_words = kNoallocCounterWords;
    const size_t part_off = kNoallocCounterWords * sizeof(int32_t);
    ws.part = reinterpret_cast<float*>(base + part_off);
    ws.part_floats = (GSP_NOALLOC_SCRATCH_BYTES - part_off) / sizeof(float);
    return attention_launch(ctx, pool, layer, n_heads, q_dev, out_dev, attn_scale, sink_logit, &ws);
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
    s.n_bt_ids = n_block_ids;
    int rc = gsp_step_pack(ctx, pool, &s);
    if (rc) return rc;
    return gsp_attention_step(ctx, pool, stage_layer, n_heads, q_dev, out_dev, attn_scale, sink_logit);
}

}  // extern "C"
