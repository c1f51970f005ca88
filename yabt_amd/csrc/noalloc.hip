// yabt_hist_noalloc: yabt_hist for callers that cannot allocate device
// memory -- code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc.  The caller passes the inputs and the outputs; the
// scratch that yabt_hist takes from its workspace argument (the quantisation
// record and the gather job) lives in the file-scope array `scratch` below,
// one copy per device, held until the process ends.
//
// Host code never passes `scratch` itself to a kernel: in host code that name
// is a stand-in, not a device address.  The device address of each device's
// copy is looked up once, with that device current, by hipGetSymbolAddress,
// and kept in `g_scratch[device]`.
//
// Every call on one device shares that device's array, which keeps the last
// call's contents; each call clears what must start at zero (by kernels, not
// memsets, so the call can be captured in a graph).  Calls that overlap on one
// device -- on two streams, or from two host threads -- race on the array.

#include "common.h"
#include "hist.h"
#include "host.h"
#include "yabt_hip.h"

#include <mutex>

namespace yabt {
namespace {

// The quantisation record and the gather job, each in its own 256-byte slot
// (the layout yabt_hist carves from its workspace).  The size does not
// depend on n or F.
constexpr size_t NOALLOC_SCRATCH_BYTES = 512;
static_assert(sizeof(Quant) <= 256 && sizeof(HistJob) <= 256, "scratch slots hold one record each");

__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES];   // device address of `scratch` per device, nullptr until looked up

// The current device's scratch address (looked up on its first call).
int scratch_of_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "yabt_hist_noalloc: current device");
    if (dev < 0 || dev >= MAX_DEVICES) return fail(-2, "yabt_hist_noalloc: device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_fail(e, "yabt_hist_noalloc: scratch address");
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace
}  // namespace yabt

using namespace yabt;

extern "C" {

int yabt_hist_noalloc(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                      const float* grad, const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m,
                      int64_t* out, int32_t* out_shifts, hipStream_t stream) {
    if (yabt_hist_workspace_bytes() > NOALLOC_SCRATCH_BYTES)
        return fail(-2, "yabt_hist_noalloc: yabt_hist's workspace exceeds the 512-byte scratch");
    void* ws = nullptr;
    if (int rc = scratch_of_current_device(&ws)) return rc;
    return hist_enqueue(bins_fm, ld_fm, bins_rm, ld_rm, grad, hess, n, F, rows, m, ws, out, out_shifts, stream,
                        "yabt_hist_noalloc");
}

}  // extern "C"
