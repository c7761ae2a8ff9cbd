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

using gsp::DecodeUnit;
using gsp::PrefillTile;
namespace {

// Packed step layout, in int32 elements from the start of the staging buffer.
enum : int {
    kHdrRows = 0,
    kHdrTotalQ,
    kHdrPages,
    kHdrUnits,
    kHdrTarget,
    kHdrSlots,
    kHdrMaxId,
    kHdrPairsSplit,
    kHdrHeadsKv,
    kHdrTiles,
    kHdrBins,
    kHdrWords = 16
};

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
        count[2 * ((size_t)base + 1) + sp] += (int64_t)extra * heads_kv;
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
    int32_t* d_mmcnt = nullptr;  // one-launch Q8_0 form: per-tile counters, zero between launches
    size_t d_mmcnt_words = 0;
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

    // Split size chosen for the last step shape (reused while the work drifts < 3%).
    int32_t cached_target = 0;
    int64_t cached_tasks = 0;
    int32_t cached_heads_kv = 0;
    int64_t cached_queries = 0;
    int64_t cached_bins = 0;

    // Host scratch reused across steps.
    std::vector<DecodeUnit> units;    // in the order they were built
    std::vector<int32_t> unit_order;  // unit indices, longest first (stable)
    std::vector<int32_t> unit_place;  // unit indices in their packed order (assign_bins)
    std::vector<int32_t> len_count;   // counting sort of unit_order
    std::vector<int32_t> stage_host;  // the step image, built in cached memory, then copied to the pinned slot
    std::vector<int32_t> bin_units;   // [num_bins + 1] offsets of each bin's units after its first
    std::vector<int32_t> unit_bin;
    std::vector<std::pair<int64_t, int32_t>> bin_heap;
    std::vector<int32_t> bin_cursor;
    std::vector<int64_t> bin_load;
    std::vector<PrefillTile> tiles;
    std::vector<gsp::PrefillSplitItem> split_items;
    std::vector<int32_t> q_ctx;
    std::vector<int32_t> query_pages;
    std::vector<int64_t> sim_count, sim_heap;
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
    if (ctx->part) (void)hipFree(ctx->part);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->d_records) (void)hipFree(ctx->d_records);
    if (ctx->aux_done) (void)hipEventDestroy(ctx->aux_done);
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

int check_rope_args(const gsp_pool* pool, int32_t n_heads, float freq_base, int32_t style, const float* q_dev) {
    if (n_heads < 0) return gsp::fail(GSP_E_INVALID_ARG, "nHeads must be >= 0 (got %d)", n_heads);
    if (n_heads > 0 && !q_dev) return gsp::fail(GSP_E_INVALID_ARG, "q is NULL with nHeads %d", n_heads);
    if (style != GSP_ROPE_PAIRS && style != GSP_ROPE_HALVES)
        return gsp::fail(GSP_E_INVALID_ARG, "unknown RoPE pairing %d", style);
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base))
        return gsp::fail(GSP_E_INVALID_ARG, "RoPE frequency base must be positive and finite");
    const gsp_pool_desc& d = pool->desc;
    if (d.head_dim % 2 != 0 || d.head_dim > 2 * gsp::kRopeMaxHalf)
        return gsp::fail(GSP_E_UNSUPPORTED, "RoPE needs an even headDim <= %d (got %d)", 2 * gsp::kRopeMaxHalf, d.head_dim);
    return GSP_OK;
}

// RoPE then Store of n tokens whose positions, block ids and slots are already on the device.
int rope_store_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* d_pos,
                      const int32_t* d_blocks, const int32_t* d_slots, int32_t n_heads, float freq_base,
                      int32_t style, float* q_dev, const float* k_dev, const float* v_dev) {
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
    a.log2_base = std::log2((double)freq_base);
    a.n = n;
    a.n_heads = n_heads;
    a.n_kv = d.heads_kv;
    a.head_dim = d.head_dim;
    a.v_head_dim = d.v_head_dim;
    a.style = style;
    return check_hip(gsp::launch_rope_write(d.kv_dtype == GSP_KV_F16, a, ctx->stream), "rope_write launch");
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

int gsp_rope_write_tokens(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n, const int32_t* positions,
                          const int32_t* block_ids, const int32_t* slots, int32_t n_heads, float freq_base,
                          int32_t style, float* q_dev, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    if (!ctx || !pool) return gsp::fail(GSP_E_INVALID_ARG, "ctx/pool is NULL");
    if (n < 0) return gsp::fail(GSP_E_INVALID_ARG, "n must be >= 0 (got %d)", n);
    if (n == 0) return GSP_OK;
    if (!positions || !block_ids || !slots || !k_dev || !v_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    int rc = check_rope_args(pool, n_heads, freq_base, style, q_dev);
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
    return rope_store_tokens(ctx, pool, layer, n, ctx->d_aux, ctx->d_aux + n, ctx->d_aux + 2 * (size_t)n, n_heads,
                             freq_base, style, q_dev, k_dev, v_dev);
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

int gsp_rope_write_step(gsp_ctx* ctx, gsp_pool* pool, int32_t layer, int32_t n_heads, float freq_base, int32_t style,
                        float* q_dev, const float* k_dev, const float* v_dev) {
    gsp::clear_error();
    int rc = check_write_step(ctx, pool, layer, k_dev, v_dev);
    if (rc) return rc;
    rc = check_rope_args(pool, n_heads, freq_base, style, q_dev);
    if (rc) return rc;
    const int32_t n = ctx->info.total_q;
    if (n == 0) return GSP_OK;
    bool cap = false;
    rc = step_begin(ctx, &cap);
    if (rc) return rc;
    const int32_t* wr = ctx->d_step + ctx->off_wr;
    rc = rope_store_tokens(ctx, pool, layer, n, wr, wr + n, wr + 2 * (size_t)n, n_heads, freq_base, style, q_dev,
                           k_dev, v_dev);
    const int rd = step_done(ctx, cap);
    return rc ? rc : rd;
}

// Q8_0 products with at least this many outputs (batch x out_dim) take the fp16
// path: measured faster from Qwen2.5-7B's 3584 x 3584 projection at 64 rows
// (229376 outputs: 27.8 vs 31.2 us) upwards, slower for 8192 x 8192 at 16 rows
// (131072 outputs: 57.5 vs 51 us) and 3584 x 512 at 64 rows (21.5 vs 16.2 us).
constexpr int64_t kMatmulF16MinOutputs = 196608;
// Q8_0 products of at most 64 batch rows with at least this many outputs take
// the small-batch fp16 form: measured faster than the other two forms from
// 8192 x 8192 at 16 rows (131072 outputs: 40.6 vs 43.7 us) and Qwen2.5-7B's
// 3584 x 3584 at 64 rows (22.1 vs 24.3 us), slower for 896 x 896 at 8 rows
// (7168 outputs: 15.8 vs 6.9 us), whose product is too small to fill the chip.
constexpr int64_t kMatmulSmallMinOutputs = 65536;

int gsp_matmul_batch(gsp_ctx* ctx, int32_t w_type, const void* w_dev, const float* x_dev, float* y_dev,
                     int32_t in_dim, int32_t out_dim, int32_t batch) {
    gsp::clear_error();
    if (!ctx) return gsp::fail(GSP_E_INVALID_ARG, "ctx is NULL");
    if (in_dim < 0 || out_dim < 0 || batch < 0)
        return gsp::fail(GSP_E_INVALID_ARG, "negative size (inDim %d, outDim %d, batch %d)", in_dim, out_dim, batch);
    if (batch == 0 || out_dim == 0) return GSP_OK;
    if (!w_dev || !x_dev || !y_dev) return gsp::fail(GSP_E_INVALID_ARG, "NULL argument");
    if (w_type != GSP_WTYPE_F32 && w_type != GSP_WTYPE_Q8_0)
        return gsp::fail(GSP_E_UNSUPPORTED, "weight type %d: only F32 (%d) and Q8_0 (%d) are supported", w_type,
                         GSP_WTYPE_F32, GSP_WTYPE_Q8_0);
    if (in_dim == 0 || in_dim % 64 != 0)
        return gsp::fail(GSP_E_UNSUPPORTED, "inDim must be a positive multiple of 64 (got %d)", in_dim);
    const uintptr_t walign = w_type == GSP_WTYPE_F32 ? 16 : 4;
    if (reinterpret_cast<uintptr_t>(w_dev) % walign != 0 || reinterpret_cast<uintptr_t>(x_dev) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(y_dev) % 4 != 0)
        return gsp::fail(GSP_E_INVALID_ARG, "weights must be %d-byte aligned, x 16-byte aligned, y 4-byte aligned",
                         (int)walign);
    int rc = set_device(ctx);
    if (rc) return rc;
    if (w_type == GSP_WTYPE_Q8_0 && batch <= 64 && (int64_t)batch * out_dim >= kMatmulSmallMinOutputs &&
        (in_dim / 64 + gsp::matmul_small_chunks(batch) - 1) / gsp::matmul_small_chunks(batch) <=
            gsp::matmul_small_max_splits(batch)) {
        // Small batches: about two workgroups (64 weight rows, every batch row)
        // per CU, K cut into ranges whose weights fit the workgroup's LDS, and
        // no more ranges than the merge holds.  The partial offsets are 32-bit.
        const int64_t chunks = in_dim / 64;
        const int64_t tiles = (out_dim + 63) / 64;
        const int64_t lo = (chunks + gsp::matmul_small_chunks(batch) - 1) / gsp::matmul_small_chunks(batch);
        const int64_t want = (2 * (int64_t)std::max(1, ctx->num_cus) + tiles - 1) / tiles;
        int64_t splits = std::max(lo, std::min({want, (int64_t)gsp::matmul_small_max_splits(batch), chunks}));
        const int64_t per = (chunks + splits - 1) / splits;
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
        if (!rc) rc = ensure_device(ctx, &ctx->d_mmexp, &ctx->d_mmexp_words, (size_t)batch, false);
        if (!rc && splits > 1) rc = ensure_device(ctx, &ctx->d_mm, &ctx->d_mm_floats, (size_t)splits * batch * tiles * 64, false);
        if (!rc && splits > 1) rc = ensure_device(ctx, &ctx->d_mmcnt, &ctx->d_mmcnt_words, (size_t)tiles, true);
        if (rc) return rc;
        a.xh = ctx->d_mmx;  // x in tile order, both halves
        a.xl = ctx->d_mmx;
        a.xexp = ctx->d_mmexp;
        a.split_out = splits > 1 ? ctx->d_mm : nullptr;
        a.counters = splits > 1 ? ctx->d_mmcnt : nullptr;
        return check_hip(gsp::launch_matmul_q8_small(a, ctx->stream), "matmul launch");
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
    if (w_type == GSP_WTYPE_Q8_0 && (int64_t)batch * out_dim >= kMatmulF16MinOutputs) {
        // Large Q8_0 products run on the fp16 matrix cores with x as scaled fp16
        // pairs; below the threshold the pre-pass launch costs more than it saves.
        const size_t halves = (size_t)batch * in_dim;
        rc = ensure_device(ctx, &ctx->d_mmx, &ctx->d_mmx_halves, 2 * halves, false);
        if (!rc) rc = ensure_device(ctx, &ctx->d_mmexp, &ctx->d_mmexp_words, (size_t)batch, false);
        if (rc) return rc;
        a.xh = ctx->d_mmx;
        a.xl = ctx->d_mmx + halves;
        a.xexp = ctx->d_mmexp;
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
static int32_t assign_bins(gsp_ctx* ctx, int64_t bins_max, bool pair) {
    const std::vector<int32_t>& ord = ctx->unit_order;
    const size_t n = ord.size();
    const int32_t nb = (int32_t)std::min<int64_t>(bins_max, (int64_t)n);
    ctx->bin_units.assign((size_t)nb + 1, 0);
    if (nb == 0) return 0;
    pair = pair && nb == bins_max && nb % 2 == 0;
    const int32_t nl = pair ? nb / 2 : nb;  // bins of the LPT
    auto& heap = ctx->bin_heap;
    heap.clear();
    for (int32_t b = 0; b < nl; ++b) heap.emplace_back(0, b);
    const std::greater<std::pair<int64_t, int32_t>> later;
    std::make_heap(heap.begin(), heap.end(), later);
    ctx->unit_bin.resize(n);
    auto& count = ctx->bin_cursor;
    count.assign((size_t)nl, 0);
    for (size_t i = 0; i < n; ++i) {
        const DecodeUnit& u = ctx->units[(size_t)ord[i]];
        std::pop_heap(heap.begin(), heap.end(), later);
        const int32_t b = heap.back().second;
        ctx->unit_bin[i] = b;
        count[(size_t)b] += 1;
        heap.back().first += unit_cost(u.page_end - u.page_begin, (u.split_info >> 16) > 1);
        std::push_heap(heap.begin(), heap.end(), later);
    }
    if (pair) {
        for (int32_t b = 0; b < nl; ++b)
            if (count[(size_t)b] < 2) return assign_bins(ctx, bins_max, false);
        auto& load = ctx->bin_load;
        load.assign((size_t)nb, 0);
        for (int pass = 0; pass < 2; ++pass)
            for (size_t i = 0; i < n; ++i) {
                const DecodeUnit& u = ctx->units[(size_t)ord[i]];
                const bool split = (u.split_info >> 16) > 1;
                if (split != (pass == 0)) continue;
                const int32_t c = ctx->unit_bin[i];
                const int32_t w = load[(size_t)c] <= load[(size_t)(c + nl)] ? c : c + nl;
                ctx->unit_bin[i] = w;
                load[(size_t)w] += unit_cost(u.page_end - u.page_begin, split);
            }
        for (size_t i = 0; i < n; ++i) ctx->bin_units[(size_t)ctx->unit_bin[i] + 1] += 1;
    } else {
        for (int32_t b = 0; b < nb; ++b) ctx->bin_units[(size_t)b + 1] = count[(size_t)b];
    }
    // bin_units[b + 1] holds bin b's unit count: its first unit goes to slot b,
    // the rest to the bin's run after the nb first units.
    ctx->bin_units[0] = nb;
    for (int32_t b = 0; b < nb; ++b) ctx->bin_units[(size_t)b + 1] += ctx->bin_units[(size_t)b] - 1;
    auto& cursor = ctx->bin_cursor;
    cursor.assign((size_t)nb, -1);  // -1: the bin's first unit is still to place
    ctx->unit_place.resize(n);
    for (int pass = 0; pass < 2; ++pass) {
        const bool want_split = pass == 0;
        for (size_t i = 0; i < n; ++i) {
            const DecodeUnit& u = ctx->units[(size_t)ord[i]];
            if (((u.split_info >> 16) > 1) != want_split) continue;
            const int32_t b = ctx->unit_bin[i];
            int32_t& cur = cursor[(size_t)b];
            if (cur < 0) {
                ctx->unit_place[(size_t)b] = ord[i];
                cur = ctx->bin_units[(size_t)b];
            } else {
                ctx->unit_place[(size_t)cur++] = ord[i];
            }
        }
    }
    return nb;
}

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
    const int32_t B = desc->num_rows;
    if (B < 0) return gsp::fail(GSP_E_INVALID_ARG, "num_rows must be >= 0 (got %d)", B);
    if (desc->max_seq_len <= 0)
        return gsp::fail(GSP_E_INVALID_ARG, "maxSeqLen must be positive (got %d)", desc->max_seq_len);
    if (B > 0 && (!desc->positions || !desc->token_counts || !desc->bt_offsets || !desc->bt_ids))
        return gsp::fail(GSP_E_INVALID_ARG, "positions/token_counts/bt_offsets/bt_ids must not be NULL");
    const int32_t L = desc->max_seq_len;
    const int32_t H = pd.heads_kv;
    const int32_t bs = pd.block_size;
    // Prefill tiles serve 16-token pages of equal K and V widths 64 or 128;
    // rows of other pools run as per-query decode units.
    const bool tileable = bs == 16 && pd.head_dim == pd.v_head_dim && (pd.head_dim == 64 || pd.head_dim == 128);

    // Pass 1: validate rows (the reference's throws, PagedAttentionKernel.cs:34-39,
    // plus the table and pool bounds) and size the packed arrays.
    int64_t total_q = 0, packed_pages = 0, kv_tokens = 0, pair_pages = 0, max_pages = 0;
    bool any_tiles = false;
    if (desc->n_bt_ids < 0) return gsp::fail(GSP_E_INVALID_ARG, "n_bt_ids must be >= 0 (got %d)", desc->n_bt_ids);
    // The CSR must stay inside the caller's id array: every row span is read
    // through bt_offsets, so they are checked before any id is.
    for (int32_t b = 0; b < B; ++b) {
        const int32_t o0 = desc->bt_offsets[b], o1 = desc->bt_offsets[b + 1];
        if (o0 < 0 || o1 < o0 || o1 > desc->n_bt_ids)
            return gsp::fail(GSP_E_INVALID_ARG, "row %d: bt_offsets [%d, %d) outside [0, n_bt_ids = %d] or decreasing",
                             b, o0, o1, desc->n_bt_ids);
    }
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
        const int64_t total_last = ql > 0 ? std::min<int64_t>(tc, (int64_t)pos + ql) : 0;
        const int64_t pages = (total_last + bs - 1) / bs;
        if (pages > span)
            return gsp::fail(GSP_E_INVALID_ARG, "row %d: %lld tokens need %lld blocks but the table holds %d", b,
                             (long long)total_last, (long long)pages, span);
        const int32_t* ids = desc->bt_ids + desc->bt_offsets[b];
        for (int64_t i = 0; i < pages; ++i)
            if (ids[i] < 0 || ids[i] >= pd.total_blocks)
                return gsp::fail(GSP_E_INVALID_ARG, "row %d: block id %d out of range [0, %d)", b, ids[i],
                                 pd.total_blocks);
        total_q += ql;
        packed_pages += pages;
        kv_tokens += total_last;
        if (row_is_tiled(ctx->prefill_path, ql, tileable)) {  // tiles, not split-KV units
            any_tiles = any_tiles || tc > 0;
            continue;
        }
        max_pages = std::max(max_pages, pages);
        for (int32_t i = 0; i < ql; ++i) {
            const int64_t tot = std::min<int64_t>(tc, (int64_t)pos + i + 1);
            pair_pages += (tot + bs - 1) / bs;
        }
    }
    if (total_q > INT32_MAX / 4 || packed_pages > INT32_MAX / 4 || pair_pages * H > INT32_MAX / 2)
        return gsp::fail(GSP_E_INVALID_ARG, "step too large");

    // Pass 2: split-KV units.  Each query token is cut into nsplit near-equal
    // page ranges of at most `target` pages; a unit is one (query token, KV
    // head, page range) and one workgroup.  Units are sorted longest first, so
    // in-order dispatch schedules them longest-processing-time first.
    const int64_t T = pair_pages * H;
    // A pair is cut into at most kMaxSplits pieces.
    const int64_t min_target = std::max<int64_t>(1, (max_pages + gsp::kMaxSplits - 1) / gsp::kMaxSplits);
    // Default grid: two workgroups per CU, bins balanced per CU (assign_bins).
    // A step that also has prefill tiles runs them beside the decode units
    // (gsp_attention_step): the HBM-bound decode grid then takes one
    // workgroup per four CUs and leaves the other slots to the matrix-bound
    // tiles, which take several times longer (config 4 measured 428 us this
    // way, against 452 us with one per two CUs and 487 us with one per CU).
    const bool pair_cus = ctx->decode_bins_override <= 0 && !any_tiles;
    const int64_t bins_max = ctx->decode_bins_override > 0 ? (int64_t)ctx->decode_bins_override
                             : pair_cus                    ? (int64_t)kDecodeBinsPerCu * std::max(1, ctx->num_cus)
                                                           : (int64_t)std::max(1, ctx->num_cus / 4);
    const int64_t sim_bins = pair_cus ? bins_max / kDecodeBinsPerCu : bins_max;
    int64_t target = 1;
    if (T > 0) {
        if (ctx->split_pages_override > 0) {
            target = std::max<int64_t>(ctx->split_pages_override, min_target);
        } else if (max_pages <= kWholePairMaxPages && T <= kUnderloadPagesPerBin * bins_max) {
            target = std::max<int64_t>(1, max_pages);  // whole pairs
        } else if (ctx->cached_target > 0 && ctx->cached_heads_kv == H && ctx->cached_queries == total_q &&
                   ctx->cached_bins == bins_max && T * 100 >= ctx->cached_tasks * 97 &&
                   T * 100 <= ctx->cached_tasks * 103) {
            target = std::max<int64_t>(ctx->cached_target, min_target);  // engine steps drift slowly
        } else {
            ctx->query_pages.clear();
            for (int32_t b = 0; b < B; ++b) {
                const int32_t ql = desc->q_lens ? desc->q_lens[b] : 1;
                if (row_is_tiled(ctx->prefill_path, ql, tileable)) continue;
                for (int32_t i = 0; i < ql; ++i) {
                    const int64_t tot = std::min<int64_t>(desc->token_counts[b], (int64_t)desc->positions[b] + i + 1);
                    if (tot > 0) ctx->query_pages.push_back((int32_t)((tot + bs - 1) / bs));
                }
            }
            int64_t best_cost = INT64_MAX;
            for (int32_t cand : kSplitCandidates) {
                if (cand < min_target) continue;
                if (T / cand > 16 * bins_max) continue;  // far too many units to be competitive
                const int64_t c = simulate_split(ctx->query_pages, H, cand, sim_bins, ctx->sim_count, ctx->sim_heap);
                if (c <= best_cost) {  // ties go to the larger split (fewer units)
                    best_cost = c;
                    target = cand;
                }
                if (cand >= max_pages) break;  // larger candidates give the same units
            }
            ctx->cached_target = (int32_t)target;
            ctx->cached_tasks = T;
            ctx->cached_heads_kv = H;
            ctx->cached_queries = total_q;
            ctx->cached_bins = bins_max;
        }
    }
    ctx->units.clear();
    ctx->tiles.clear();
    ctx->split_items.clear();
    ctx->q_ctx.assign((size_t)total_q, 0);
    // fp32 tiles read split records (one per page pair of each tiled row and
    // KV head) unless the caller asked the tiles to split their own pages.
    const bool records = tileable && pd.kv_dtype == GSP_KV_F32 && ctx->prefill_split == GSP_SPLIT_RECORDS;
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
            if (row_is_tiled(ctx->prefill_path, ql, tileable)) {
                // Causal tiles of 16 query tokens; a row with TokenCount 0 has
                // total 0 for every token and gets none (out left untouched).
                for (int32_t i = 0; i < ql; ++i)
                    ctx->q_ctx[qi + i] = (int32_t)std::min<int64_t>(tc, (int64_t)pos + i + 1);
                if (tc > 0) {
                    // The row's page pairs: every tile of the row reads a prefix of them.
                    const int32_t row_pairs = (int32_t)(((total_last + bs - 1) / bs + 1) / 2);
                    const int64_t rec_row = n_records;
                    if (records) {
                        for (int32_t kvh = 0; kvh < H; ++kvh)
                            ctx->split_items.push_back(gsp::PrefillSplitItem{
                                (int32_t)bt_base, (int32_t)total_last, kvh, (int32_t)(rec_row + (int64_t)kvh * row_pairs)});
                        n_records += (int64_t)H * row_pairs;
                        split_max_pairs = std::max(split_max_pairs, row_pairs);
                    }
                    for (int32_t t0 = 0; t0 < ql; t0 += gsp::kPrefillTileTokens) {
                        PrefillTile t;
                        t.qi0 = (int32_t)(qi + t0);
                        t.bt_base = (int32_t)bt_base;
                        t.pos0 = pos + t0;
                        t.ntok = std::min(gsp::kPrefillTileTokens, ql - t0);
                        t.token_count = tc;
                        const int64_t last = std::min<int64_t>(tc, (int64_t)t.pos0 + t.ntok);
                        t.pages = (int32_t)((last + bs - 1) / bs);
                        for (int32_t kvh = 0; kvh < H; ++kvh) {
                            t.kvh = kvh;
                            t.rec0 = records ? (int32_t)(rec_row + (int64_t)kvh * row_pairs) : 0;
                            ctx->tiles.push_back(t);
                        }
                    }
                    for (int32_t i = 0; i < ql; ++i) tiled_pairs += ctx->q_ctx[qi + i];
                    tiled_queries += ql;
                }
                qi += ql;
                bt_base += (total_last + bs - 1) / bs;
                continue;
            }
            for (int32_t i = 0; i < ql; ++i, ++qi) {
                const int32_t tot = (int32_t)std::min<int64_t>(tc, (int64_t)pos + i + 1);
                ctx->q_ctx[qi] = tot;
                if (tot <= 0) continue;
                const int32_t pages = (tot + bs - 1) / bs;
                const int32_t nsplit = (int32_t)std::min<int64_t>((pages + target - 1) / target, gsp::kMaxSplits);
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
                        for (int w = 0; w < gsp::kDecodeWaves; ++w) {
                            const int32_t p = u.page_begin + w;
                            const int32_t p2 = p + gsp::kDecodeWaves;
                            u.first_blk[w] = p < u.page_end ? row_ids[p] : -1;
                            u.second_blk[w] = p2 < u.page_end ? row_ids[p2] : -1;
                        }
                        ctx->units.push_back(u);
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
        for (const DecodeUnit& u : ctx->units) max_len = std::max(max_len, u.page_end - u.page_begin);
        auto& cnt = ctx->len_count;
        cnt.assign((size_t)max_len + 2, 0);
        for (const DecodeUnit& u : ctx->units) cnt[(size_t)(max_len - (u.page_end - u.page_begin)) + 1] += 1;
        for (size_t l = 1; l < cnt.size(); ++l) cnt[l] += cnt[l - 1];
        ctx->unit_order.resize(ctx->units.size());
        for (size_t i = 0; i < ctx->units.size(); ++i) {
            const DecodeUnit& u = ctx->units[i];
            ctx->unit_order[(size_t)cnt[(size_t)(max_len - (u.page_end - u.page_begin))]++] = (int32_t)i;
        }
    }
    if (ctx->split_items.size() > kMaxSplitItems) {  // the tiles split their own pages
        ctx->split_items.clear();
        n_records = 0;
        split_max_pairs = 0;
    }
    std::stable_sort(ctx->tiles.begin(), ctx->tiles.end(),
                     [](const PrefillTile& x, const PrefillTile& y) { return x.pages > y.pages; });
    const int32_t n_bins = assign_bins(ctx, bins_max, pair_cus);

    // Pass 3: write the staging buffer and upload it with one copy.
    const size_t n_units = ctx->units.size();
    const size_t n_tiles = ctx->tiles.size();
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
    const size_t n_split = ctx->split_items.size();
    const size_t off_split = off;
    off += n_split * (sizeof(gsp::PrefillSplitItem) / sizeof(int32_t));
    const size_t off_bins = off;
    off += (size_t)n_bins + 1;
    const size_t words = off;
    const size_t words16 = align_up(words, 4);  // the upload moves 16-byte words

    int rc = set_device(ctx);
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
    if (!rc && slots > 0)
        rc = ensure_device(ctx, &ctx->part, &ctx->part_floats,
                           (size_t)slots * gsp::kMaxGroupMfma * (size_t)(pd.v_head_dim + 2), false);
    if (!rc && slots > 0)
        rc = ensure_device(ctx, &ctx->counters, &ctx->counter_words, (size_t)total_q * H, true);
    // The split records, so that a captured gsp_attention_step never grows them.
    if (!rc && n_records > 0)
        rc = ensure_device(ctx, &ctx->d_records, &ctx->d_records_bytes,
                           (size_t)n_records * (size_t)gsp::prefill_record_bytes(pd.head_dim), false);
    if (rc) return rc;

    // The step image is written in cached host memory and copied into the
    // pinned slot in one pass: element-wise stores straight into the pinned
    // buffer measured several times slower.
    ctx->stage_host.resize(words);
    int32_t* st = ctx->stage_host.data();
    std::memset(st, 0, kHdrWords * sizeof(int32_t));
    int32_t max_id = -1;
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
            for (int64_t i = 0; i < pages; ++i) {
                ids[w++] = src[i];
                max_id = std::max(max_id, src[i]);
            }
            rows[b + 1] = (int32_t)w;
            // A query token at p < TokenCount has its slot in the packed pages
            // (p < total_last); the reference stores its K/V there before
            // attending (PagedTransformerRunner.cs:620-634, :437-452).
            for (int32_t i = 0; i < ql; ++i, ++qi) {
                const int64_t p = (int64_t)pos + i;
                wr_pos[qi] = (int32_t)p;
                const bool has = p < tc;
                wr_blk[qi] = has ? src[p / bs] : -1;
                wr_slot[qi] = has ? (int32_t)(p % bs) : 0;
            }
        }
    }
    if (total_q) std::memcpy(st + off_ctx, ctx->q_ctx.data(), (size_t)total_q * sizeof(int32_t));
    {
        DecodeUnit* dst = reinterpret_cast<DecodeUnit*>(st + off_units);
        for (size_t j = 0; j < n_units; ++j) dst[j] = ctx->units[(size_t)ctx->unit_place[j]];
    }
    if (n_tiles) std::memcpy(st + off_tiles, ctx->tiles.data(), n_tiles * sizeof(PrefillTile));
    if (n_split) std::memcpy(st + off_split, ctx->split_items.data(), n_split * sizeof(gsp::PrefillSplitItem));
    std::memcpy(st + off_bins, ctx->bin_units.data(), ((size_t)n_bins + 1) * sizeof(int32_t));
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

    // One copy for the whole step, on the context's stream (behind the
    // kernels that read this slot's previous step), then the event that frees
    // the pinned buffer.  The pad words up to a 16-byte word are zeroed.
    std::memcpy(ctx->staging[slot], st, words * sizeof(int32_t));
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

    ctx->off_rows = off_rows;
    ctx->off_ids = off_ids;
    ctx->off_ctx = off_ctx;
    ctx->off_wr = off_wr;
    ctx->off_units = off_units;
    ctx->off_tiles = off_tiles;
    ctx->off_split = off_split;
    ctx->off_bins = off_bins;
    ctx->num_split_items = (int32_t)n_split;
    ctx->split_max_pairs = split_max_pairs;
    ctx->num_records = n_records;
    ctx->records_head_dim = n_records > 0 ? pd.head_dim : 0;
    ctx->num_bins = n_bins;
    ctx->max_id = max_id;
    ctx->num_slots = (int32_t)slots;
    ctx->num_units = (int32_t)n_units;
    ctx->num_tiles = (int32_t)n_tiles;
    ctx->step_heads_kv = H;
    ctx->step_blocks = pd.total_blocks;
    ctx->step_block_size = bs;
    ctx->step_tileable = tileable;
    ctx->info.num_rows = B;
    ctx->info.total_q = (int32_t)total_q;
    ctx->info.packed_pages = (int32_t)packed_pages;
    ctx->info.heads_kv = H;
    ctx->info.decode_units = (int32_t)n_units;
    ctx->info.split_pairs = (int32_t)pairs_split;
    ctx->info.partial_slots = (int32_t)slots;
    ctx->info.pages_per_split = (int32_t)target;
    ctx->info.kv_tokens = kv_tokens;
    ctx->info.staging_bytes = (int64_t)(words * sizeof(int32_t));
    ctx->info.prefill_tiles = (int32_t)n_tiles;
    ctx->info.prefill_queries = (int32_t)tiled_queries;
    ctx->info.prefill_pairs = tiled_pairs;
    ctx->info.decode_bins = n_bins;
    ctx->info.split_records = (int32_t)n_records;
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
    // The reference GPU runner's domain (CudaPagedTransformerRunner.cs:408-412).
    if (d.head_dim % 2 || d.v_head_dim % 2 || d.head_dim > 256 || d.v_head_dim > 256)
        return gsp::fail(GSP_E_UNSUPPORTED, "headDim (%d) and vHeadDim (%d) must be even and at most 256", d.head_dim,
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
         d.block_size != gsp::kBlockSize))
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
    a.block_stride = pool->block_stride_k;
    a.layer_offset = (int64_t)layer * pool->layer_stride_k;
    a.head_stride = pool->head_stride_k;
    a.v_block_stride = pool->block_stride_v;
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
    a.block_size = d.block_size;
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
