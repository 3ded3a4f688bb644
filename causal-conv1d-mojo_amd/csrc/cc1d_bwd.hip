// cc1d_bwd.hip -- backward entry points: dispatch on the dtype code to the
// per-dtype launchers (cc1d_bwd_kernels.hpp, instantiated by
// cc1d_bwd_{fp16,bf16,fp32}.hip), and the allocation-free typed backward
// with its static device scratch.
#include <mutex>

#include "cc1d_internal.hpp"

namespace cc1d {

int launch_bwd(const cc1d_bwd_params& p, hipStream_t stream) {
    return with_dtype(p.dtype, [&](auto tag) { return launch_bwd_dtype<decltype(tag)>(p, stream); });
}

int launch_bwd_typed(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream) {
    return with_dtype(p.dtype, [&](auto tag) { return launch_bwd_typed_dtype<decltype(tag)>(p, g, stream); });
}

int64_t bwd_workspace_floats(const cc1d_bwd_params& p) {
    int64_t n = -1;
    with_dtype(p.dtype, [&](auto tag) {
        n = bwd_workspace_floats_dtype<decltype(tag)>(p);
        return (int)CC1D_OK;
    });
    return n;
}

// ---- allocation-free typed backward ------------------------------------
//
// The partial-sum workspace of cc1d_bwd_typed_noalloc lives in this
// file-scope device array, one copy per GPU for the life of the process.
// Host code never passes `scratch` itself to a kernel (on the host the name
// stands for a host-side shadow, not a device address): each device's address
// comes from hipGetSymbolAddress, taken once per device with that device
// current, and only that address is used. The backward kernel writes every
// record the reduction reads, so nothing needs clearing between calls. Calls
// that overlap on one GPU (other streams, other threads) share the array and
// race.
static __device__ __align__(256) float scratch[kStaticWorkspaceFloats];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream); set up on the first call for that device.
int scratch_ptr(hipStream_t stream, float** out) {
    int dev = -1;
    if (stream != nullptr) {
        if (hipStreamGetDevice(stream, &dev) != hipSuccess) return CC1D_ERR_LAUNCH;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return CC1D_ERR_LAUNCH;
    }
    if (dev < 0 || dev >= kMaxDevices) return CC1D_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return CC1D_ERR_LAUNCH;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return CC1D_ERR_LAUNCH;
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || ptr == nullptr) return CC1D_ERR_LAUNCH;
        g_scratch_ptr[dev] = static_cast<float*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return CC1D_OK;
}

}  // namespace

int launch_bwd_typed_noalloc(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream) {
    if (bwd_workspace_floats(p) > kStaticWorkspaceFloats) return CC1D_ERR_SCRATCH_LIMIT;
    float* ws = nullptr;
    const int st = scratch_ptr(stream, &ws);
    if (st != CC1D_OK) return st;
    cc1d_bwd_grads gs = g;
    gs.workspace = ws;
    gs.workspace_floats = kStaticWorkspaceFloats;
    return launch_bwd_typed(p, gs, stream);
}

}  // namespace cc1d
