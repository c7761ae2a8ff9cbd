// Fixed device scratch of gsp_attention_step_noalloc: the split-KV partials
// and per-pair counters of a decode launch live in this array instead of in
// context workspace grown with hipMalloc.  Each GPU holds its own copy of the
// array (at its own address) from the moment the library's code object is
// loaded there until the process ends.
//
// On the host, `scratch` names a host-side stand-in, not a device address, so
// host code never passes it to a kernel or a copy: gsp_init looks the device
// address up once per device (with that device current) through
// hipGetSymbolAddress, and every later use goes through that pointer.
#include <atomic>
#include <mutex>

#include "../../include/glacier_paged.h"
#include "gsp_internal.h"

namespace {

static_assert(GSP_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size is a multiple of its alignment");

static __device__ __align__(256) unsigned char scratch[GSP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
// The lookup runs once per device under the mutex; the per-call read of the
// pointer (noalloc_scratch) takes no lock: the pointer is published with a
// release store and read with an acquire load, and never changes afterwards.
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];  // static storage: zero (nullptr) before any store

}  // namespace

namespace gsp {

hipError_t noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device].load(std::memory_order_acquire)) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[device].store(p, std::memory_order_release);
    return hipSuccess;
}

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    return g_scratch_ptr[device].load(std::memory_order_acquire);
}

}  // namespace gsp
