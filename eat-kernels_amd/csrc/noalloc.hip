// libkda355_noalloc.so: kda355_prefill_launch without a caller workspace, for callers that cannot allocate (code under
// graph capture with no allocator at hand, tight serving loops).  It is a library of its own so that the static
// device array below is held only by processes that load it: every GPU such a process runs the entry point on holds
// its own copy from the code object's load to the end of the process.  The host never uses the array's name as an
// address: the device address of the current device's copy comes from hipGetSymbolAddress, once per device.  Every
// kernel of libkda355 writes each workspace word it reads earlier in the same call (the chunk kernel writes the pieces'
// states, transitions and correction operands; the scan and compose passes read them after it), so nothing has to
// start at zero and what an earlier call left there is never read.  Calls that overlap on one GPU (two streams, or
// two threads) share the array and race.
#include <mutex>

#include "common.h"

static __device__ __align__(256) unsigned char scratch[KDA355_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {nullptr};

// the device address of the current device's scratch copy (resolved at the first call on that device)
int scratch_address(void** out) {
    int dev = -1;
    const hipError_t e0 = hipGetDevice(&dev);
    if (e0 != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        kda355::set_error("prefill_noalloc: hipGetDevice failed (%s, device %d)", hipGetErrorString(e0), dev);
        return KDA355_ELAUNCH;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            kda355::set_error("prefill_noalloc: hipGetSymbolAddress of the static scratch failed on device %d: %s", dev,
                              hipGetErrorString(e));
            return KDA355_ELAUNCH;
        }
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}
}  // namespace

extern "C" int kda355_prefill_launch_noalloc(const KdaPrefillArgs* a, kda355_stream_t stream) {
    KDA_CHECK_ARG(a && a->plan, "prefill_noalloc: null args or plan");
    const int64_t ws = kda355_prefill_workspace_bytes(a->plan);
    KDA_CHECK_ARG(ws >= 0, "prefill_noalloc: plan is not a kda355_prefill_plan() result");
    KDA_CHECK_ARG(a->workspace == nullptr, "prefill_noalloc: takes no workspace (it uses the library's static scratch)");
    KDA_CHECK_ARG(ws <= (int64_t)KDA355_NOALLOC_SCRATCH_BYTES,
                  "prefill_noalloc: this layout needs %lld bytes of workspace, the static scratch holds %lld "
                  "(use kda355_prefill_launch with a caller workspace)",
                  (long long)ws, (long long)KDA355_NOALLOC_SCRATCH_BYTES);
    KdaPrefillArgs b = *a;
    if (ws > 0) {
        void* ptr = nullptr;
        const int rc = scratch_address(&ptr);
        if (rc != 0) return rc;
        b.workspace = ptr;
    }
    return kda355_prefill_launch(&b, stream);
}
