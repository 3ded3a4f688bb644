// cc1d_abi.hip -- extern "C" entry points declared in include/cc1d.h.
//
// Validates the plain-pointer arguments, handles zero-size problems, and
// forwards to the kernel launchers on the caller's stream. No allocation, no
// synchronisation, no exceptions across the boundary.
#include "cc1d_internal.hpp"

using namespace cc1d;

namespace {

constexpr int64_t kMaxBlocks = (int64_t)1 << 31;

bool valid_dtype(int32_t d) { return d == CC1D_DTYPE_FP16 || d == CC1D_DTYPE_BF16 || d == CC1D_DTYPE_FP32; }
bool valid_width(int64_t w) { return w >= 2 && w <= 9; }
int esize(int32_t d) { return d == CC1D_DTYPE_FP32 ? 4 : 2; }

// Every launcher uses at most one thread per element of the largest tensor
// it touches; refuse problems whose grids would not fit.
bool grid_fits(int64_t threads) { return threads / 256 + 1 < kMaxBlocks; }

// Shared by cc1d_bwd_typed and cc1d_bwd_typed_noalloc (which ignores the workspace).
int bwd_typed_entry(const cc1d_bwd_params* p, const cc1d_bwd_grads* g, void* stream, bool noalloc) {
    if (p == nullptr || g == nullptr) return CC1D_ERR_NULL_POINTER;
    if (!valid_dtype(p->dtype)) return CC1D_ERR_DTYPE;
    if (!valid_width(p->width)) return CC1D_ERR_WIDTH;
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0) return CC1D_ERR_SHAPE;
    if (p->seq_idx != nullptr &&
        (p->initial_states != nullptr || p->dfinal_states != nullptr || p->dinitial_states != nullptr))
        return CC1D_ERR_EXCLUSIVE;
    if (p->initial_states != nullptr && p->dinitial_states == nullptr) return CC1D_ERR_NULL_POINTER;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (p->dim == 0) return CC1D_OK;
    if (g->dweight == nullptr) return CC1D_ERR_NULL_POINTER;
    if (p->batch == 0 || p->seqlen == 0) {
        // no positions: the gradients are sums over no terms
        const int64_t ws[3] = {0, g->dweight_stride[0], g->dweight_stride[1]};
        int st = launch_zero3(g->dweight, esize(p->dtype), 1, p->dim, p->width, ws, s);
        if (st == CC1D_OK && g->dbias != nullptr) {
            const int64_t bs[3] = {0, g->dbias_stride, 0};
            st = launch_zero3(g->dbias, esize(p->dtype), 1, p->dim, 1, bs, s);
        }
        if (st == CC1D_OK && p->dinitial_states != nullptr && p->batch > 0)
            st = launch_zero3(p->dinitial_states, esize(p->dtype), p->batch, p->dim, p->width - 1,
                              p->dinitial_states_stride, s);
        return st;
    }
    if (!grid_fits(p->batch * p->dim * p->seqlen)) return CC1D_ERR_SHAPE;
    if (p->x == nullptr || p->weight == nullptr || p->dout == nullptr || p->dx == nullptr)
        return CC1D_ERR_NULL_POINTER;
    // (a NULL workspace is refused by the launcher when the call needs one)
    if (noalloc) return launch_bwd_typed_noalloc(*p, *g, s);
    return launch_bwd_typed(*p, *g, s);
}

}  // namespace

extern "C" {

int cc1d_abi_version(void) { return CC1D_ABI_VERSION; }

const char* cc1d_strerror(int status) {
    switch (status) {
    case CC1D_OK: return "ok";
    case CC1D_ERR_NULL_POINTER: return "a required pointer is NULL";
    case CC1D_ERR_DTYPE: return "unsupported dtype code (expected 0=fp16, 1=bf16, 2=fp32) or element size";
    case CC1D_ERR_WIDTH: return "width must be in 2..9";
    case CC1D_ERR_SHAPE: return "invalid or too large shape";
    case CC1D_ERR_EXCLUSIVE: return "seq_idx is mutually exclusive with initial_states and final_states";
    case CC1D_ERR_STATE_LEN: return "conv_state length must be >= width - 1";
    case CC1D_ERR_LAUNCH: return "kernel launch failed";
    case CC1D_ERR_WORKSPACE: return "workspace smaller than cc1d_bwd_workspace_floats()";
    case CC1D_ERR_SCRATCH_LIMIT:
        return "problem needs more workspace than the static scratch of cc1d_bwd_typed_noalloc "
               "(CC1D_NOALLOC_WORKSPACE_FLOATS floats)";
    default: return "unknown status";
    }
}

int cc1d_fwd(const cc1d_fwd_params* p, void* stream) {
    if (p == nullptr) return CC1D_ERR_NULL_POINTER;
    if (!valid_dtype(p->dtype)) return CC1D_ERR_DTYPE;
    if (!valid_width(p->width)) return CC1D_ERR_WIDTH;
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0) return CC1D_ERR_SHAPE;
    if (p->seq_idx != nullptr && (p->initial_states != nullptr || p->final_states_out != nullptr))
        return CC1D_ERR_EXCLUSIVE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (p->batch == 0 || p->dim == 0) return CC1D_OK;
    if (!grid_fits(p->batch * p->dim * (p->seqlen > 0 ? p->seqlen : 1))) return CC1D_ERR_SHAPE;
    if (p->seqlen == 0) {
        if (p->final_states_out == nullptr) return CC1D_OK;
        return launch_zero3(p->final_states_out, esize(p->dtype), p->batch, p->dim, p->width - 1,
                            p->final_states_stride, s);
    }
    if (p->x == nullptr || p->weight == nullptr || p->out == nullptr) return CC1D_ERR_NULL_POINTER;
    return launch_fwd(*p, s);
}

int cc1d_bwd(const cc1d_bwd_params* p, void* stream) {
    if (p == nullptr) return CC1D_ERR_NULL_POINTER;
    if (!valid_dtype(p->dtype)) return CC1D_ERR_DTYPE;
    if (!valid_width(p->width)) return CC1D_ERR_WIDTH;
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0) return CC1D_ERR_SHAPE;
    if (p->seq_idx != nullptr &&
        (p->initial_states != nullptr || p->dfinal_states != nullptr || p->dinitial_states != nullptr))
        return CC1D_ERR_EXCLUSIVE;
    if (p->initial_states != nullptr && p->dinitial_states == nullptr) return CC1D_ERR_NULL_POINTER;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (p->batch == 0 || p->dim == 0) return CC1D_OK;
    if (!grid_fits(p->batch * p->dim * (p->seqlen > 0 ? p->seqlen : 1))) return CC1D_ERR_SHAPE;
    if (p->seqlen == 0) {
        // no positions: dx is empty, the accumulators receive nothing and
        // dinitial_states (a sum over no terms) is zero
        if (p->dinitial_states == nullptr) return CC1D_OK;
        return launch_zero3(p->dinitial_states, esize(p->dtype), p->batch, p->dim, p->width - 1,
                            p->dinitial_states_stride, s);
    }
    if (p->x == nullptr || p->weight == nullptr || p->dout == nullptr || p->dx == nullptr ||
        p->dweight_acc == nullptr)
        return CC1D_ERR_NULL_POINTER;
    return launch_bwd(*p, s);
}

int64_t cc1d_bwd_workspace_floats(const cc1d_bwd_params* p) {
    if (p == nullptr || !valid_dtype(p->dtype) || !valid_width(p->width)) return -1;
    if (p->batch <= 0 || p->dim <= 0 || p->seqlen <= 0) return 0;
    return bwd_workspace_floats(*p);
}

int cc1d_bwd_typed(const cc1d_bwd_params* p, const cc1d_bwd_grads* g, void* stream) {
    return bwd_typed_entry(p, g, stream, false);
}

int cc1d_bwd_typed_noalloc(const cc1d_bwd_params* p, const cc1d_bwd_grads* g, void* stream) {
    return bwd_typed_entry(p, g, stream, true);
}

int cc1d_update(const cc1d_update_params* p, void* stream) {
    if (p == nullptr) return CC1D_ERR_NULL_POINTER;
    if (!valid_dtype(p->dtype)) return CC1D_ERR_DTYPE;
    if (!valid_width(p->width)) return CC1D_ERR_WIDTH;
    if (p->batch < 0 || p->dim < 0 || p->seqlen < 0 || p->state_len < 0 || p->state_rows < 0)
        return CC1D_ERR_SHAPE;
    if (p->state_len < p->width - 1) return CC1D_ERR_STATE_LEN;
    if (p->conv_state_indices == nullptr && p->state_rows < p->batch) return CC1D_ERR_SHAPE;
    if (p->batch == 0 || p->dim == 0 || p->seqlen == 0) return CC1D_OK;
    if (!grid_fits(p->batch * p->dim)) return CC1D_ERR_SHAPE;
    if (p->x == nullptr || p->weight == nullptr || p->conv_state == nullptr || p->out == nullptr)
        return CC1D_ERR_NULL_POINTER;
    return launch_update(*p, static_cast<hipStream_t>(stream));
}

int cc1d_varlen_states(const cc1d_varlen_params* p, void* stream) {
    if (p == nullptr) return CC1D_ERR_NULL_POINTER;
    if (p->elem_bytes == 0 ? !valid_dtype(p->dtype)
                           : (p->elem_bytes != 1 && p->elem_bytes != 2 && p->elem_bytes != 4 && p->elem_bytes != 8 &&
                              p->elem_bytes != 16))
        return CC1D_ERR_DTYPE;
    if (p->total_tokens < 0 || p->dim < 0 || p->batch < 0 || p->state_len < 0) return CC1D_ERR_SHAPE;
    if (p->batch == 0 || p->dim == 0 || p->state_len == 0) return CC1D_OK;
    if (!grid_fits(p->batch * p->dim * p->state_len)) return CC1D_ERR_SHAPE;
    if (p->cu_seqlens == nullptr || p->states == nullptr || (p->x == nullptr && p->total_tokens > 0))
        return CC1D_ERR_NULL_POINTER;
    return launch_varlen_states(*p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
