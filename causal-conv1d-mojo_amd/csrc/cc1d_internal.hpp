// cc1d_internal.hpp -- host-side glue shared by the launcher translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <tuple>
#include <type_traits>

#include "cc1d.h"
#include "cc1d_device.hpp"

namespace cc1d {

// Launchers (one per kernel family). The arguments were validated by the C
// ABI layer; each returns a cc1d_status.
int launch_fwd(const cc1d_fwd_params& p, hipStream_t stream);
int launch_bwd(const cc1d_bwd_params& p, hipStream_t stream);
int launch_bwd_typed(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream);
// As launch_bwd_typed with the library's static device scratch as the
// workspace (g.workspace is ignored); CC1D_ERR_SCRATCH_LIMIT when the
// problem needs more than kStaticWorkspaceFloats.
int launch_bwd_typed_noalloc(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream);
constexpr int64_t kStaticWorkspaceFloats = CC1D_NOALLOC_WORKSPACE_FLOATS;
int64_t bwd_workspace_floats(const cc1d_bwd_params& p);
// per-dtype backward launchers (explicitly instantiated in cc1d_bwd_<dtype>.hip)
template <typename T> int launch_bwd_dtype(const cc1d_bwd_params& p, hipStream_t stream);
template <typename T>
int launch_bwd_typed_dtype(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream);
template <typename T> int64_t bwd_workspace_floats_dtype(const cc1d_bwd_params& p);
int launch_update(const cc1d_update_params& p, hipStream_t stream);
int launch_varlen_states(const cc1d_varlen_params& p, hipStream_t stream);
// element size of a varlen gather: elem_bytes, or the size of dtype when it is 0
int varlen_elem_bytes(const cc1d_varlen_params& p);

// Compile-time dispatch over the runtime dtype code / width / flags.
template <typename F> int with_dtype(int dtype, F&& f) {
    switch (dtype) {
    case CC1D_DTYPE_FP16: return f(f16{});
    case CC1D_DTYPE_BF16: return f(bf16{});
    case CC1D_DTYPE_FP32: return f(float{});
    default: return CC1D_ERR_DTYPE;
    }
}

template <typename F> int with_width(int64_t width, F&& f) {
    switch (width) {
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 5: return f(std::integral_constant<int, 5>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 7: return f(std::integral_constant<int, 7>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 9: return f(std::integral_constant<int, 9>{});
    default: return CC1D_ERR_WIDTH;
    }
}

template <typename F> int with_flag(bool flag, F&& f) {
    return flag ? f(std::true_type{}) : f(std::false_type{});
}

// Launches kernel k with the given arguments (converted to its parameter
// types) and returns the status of this launch alone: hipLaunchKernel reports
// it directly, so an error that an earlier, unrelated call left on the thread
// is neither returned as ours nor cleared. A failed launch's own error is
// taken off the thread, so it does not surface in the caller's next check.
template <typename... P, typename... A>
int launch(void (*k)(P...), dim3 grid, dim3 block, hipStream_t stream, const A&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "one argument per kernel parameter");
    std::tuple<std::decay_t<P>...> vals(args...);
    void* ptrs[sizeof...(P)];
    std::apply([&](auto&... v) {
        int i = 0;
        ((ptrs[i++] = static_cast<void*>(&v)), ...);
    }, vals);
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(k), grid, block, ptrs, 0, stream);
    if (e == hipSuccess) return CC1D_OK;
    (void)hipGetLastError();
    return CC1D_ERR_LAUNCH;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Zero-fills a (n0, n1, n2) strided tensor of `esize`-byte elements.
int launch_zero3(void* ptr, int esize, int64_t n0, int64_t n1, int64_t n2,
                 const int64_t* stride, hipStream_t stream);

}  // namespace cc1d
