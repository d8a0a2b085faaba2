// lt_noalloc.hip -- the device memory of lt_moe_forward_noalloc.
//
// Callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc) run the single-launch MoE kernel on a scratch area
// the library holds for the life of the process: `scratch` below, one copy
// per GPU (a module global, zero when the code object loads).  Its device
// address is looked up with hipGetSymbolAddress once per device, at lt_init
// with that device current, and kept in g_base: host code uses that
// address, never the array's name, which on the host is only a stand-in.
//
// Nothing in the area needs clearing per call: the kernel's hand-over words
// carry launch epochs and every launch advances all launch counters
// together (lt_moe_fused.hip).  All calls on one GPU share the area, so
// calls that overlap on one GPU (several streams or contexts) race.
#include "lt_internal.h"

#include <mutex>

namespace lt {

static __device__ __align__(256) uint8_t scratch[kFusedScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t *g_base[kMaxDevices];
}  // namespace

hipError_t noalloc_scratch(int device, uint8_t **base) {
    *base = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_base[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_base[device] = static_cast<uint8_t *>(p);
    }
    *base = g_base[device];
    return hipSuccess;
}

}  // namespace lt
