// cc1d_bwd_fp32.hip -- the backward kernels and launchers for float storage
// (one translation unit per dtype, so the three compile in parallel).
#include "cc1d_bwd_kernels.hpp"

namespace cc1d {

template int launch_bwd_dtype<float>(const cc1d_bwd_params&, hipStream_t);
template int launch_bwd_typed_dtype<float>(const cc1d_bwd_params&, const cc1d_bwd_grads&, hipStream_t);
template int64_t bwd_workspace_floats_dtype<float>(const cc1d_bwd_params&);

}  // namespace cc1d
