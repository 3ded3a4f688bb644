/*
 * cc1d.h -- C ABI of the MI355X (gfx950) depthwise causal conv1d library
 * (libcc1d_amd.so).
 *
 * Plain pointers, sizes and element strides; no torch types. Every entry
 * point enqueues its kernels on the caller's HIP stream and returns without
 * synchronising. It never allocates device memory, never synchronises the
 * device and never throws across the ABI, so a call may be captured in a HIP
 * graph. Tensors are owned by the caller; the library only borrows pointers.
 *
 * Conventions shared by all entry points
 *   - Pointers are device pointers. NULL marks an absent optional tensor.
 *   - Strides are int64 element strides (torch.Tensor.stride()).
 *   - dtype codes are those of the reference's _DTYPE_CODE
 *     (src/causal_conv1d_mojo/_dtype.py:16-20): 0 fp16, 1 bf16, 2 fp32.
 *   - Arithmetic is fp32; each output element is rounded once
 *     (round-to-nearest-even) to its storage dtype.
 *   - A zero-size problem enqueues nothing except the zero-fill that a
 *     requested final_states needs.
 *   - The return value is CC1D_OK or one of the CC1D_ERR_* codes; a code
 *     other than CC1D_OK means nothing was enqueued.
 *
 * The entry points replace the reference's per-variant CPython extension
 * entry points (paths relative to /root/reference):
 *   cc1d_fwd           <- causal_conv1d_fwd_variant, src/causal_conv1d_mojo/fwd/variant.mojo:58-131,
 *                         fed by native_fwd's 29-int tuple, src/causal_conv1d_mojo/fwd/__init__.py:11-60
 *   cc1d_bwd           <- causal_conv1d_bwd_full_variant, src/causal_conv1d_mojo/bwd_full/variant.mojo:50-144,
 *                         fed by native_bwd_full, src/causal_conv1d_mojo/bwd_full/__init__.py:11-73
 *   cc1d_bwd_typed     <- the same kernel plus the accumulator zero-fill and the casts of the
 *                         autograd backward, src/causal_conv1d_mojo/_fn.py:276-292,317-320
 *   cc1d_update        <- causal_conv1d_update_variant, src/causal_conv1d_mojo/update/variant.mojo:45-116,
 *                         fed by native_update, src/causal_conv1d_mojo/update/__init__.py:11-60
 *   cc1d_varlen_states <- causal_conv1d_varlen_states (pure torch in the reference),
 *                         src/causal_conv1d_mojo/causal_conv1d_varlen.py:29-61
 */
#ifndef CC1D_H
#define CC1D_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CC1D_ABI_VERSION 3

enum cc1d_dtype {
    CC1D_DTYPE_FP16 = 0,
    CC1D_DTYPE_BF16 = 1,
    CC1D_DTYPE_FP32 = 2
};

enum cc1d_status {
    CC1D_OK = 0,
    CC1D_ERR_NULL_POINTER = 1,      /* a required pointer (or the params struct) is NULL */
    CC1D_ERR_DTYPE = 2,             /* dtype code not in {0, 1, 2} (varlen: or elem_bytes not in {0, 1, 2, 4, 8, 16}) */
    CC1D_ERR_WIDTH = 3,             /* width outside 2..9 */
    CC1D_ERR_SHAPE = 4,             /* negative size, or a size/stride too large for the kernels */
    CC1D_ERR_EXCLUSIVE = 5,         /* seq_idx given together with initial_states or final_states
                                       (backward: or with dfinal_states / dinitial_states) */
    CC1D_ERR_STATE_LEN = 6,         /* conv_state length < width - 1 */
    CC1D_ERR_LAUNCH = 7,            /* the HIP runtime refused a kernel launch */
    CC1D_ERR_WORKSPACE = 8,         /* workspace smaller than cc1d_bwd_workspace_floats() */
    CC1D_ERR_SCRATCH_LIMIT = 9      /* cc1d_bwd_typed_noalloc: the problem needs more than
                                       CC1D_NOALLOC_WORKSPACE_FLOATS floats of workspace */
};

/* Size (fp32 elements) of the static device scratch of cc1d_bwd_typed_noalloc: 8 MiB, reserved on
   every GPU where the library's kernels are loaded, whether or not cc1d_bwd_typed_noalloc is called
   (the largest benchmark need, 8 x 2048 x 16384 fp32 at width 4, is 1,310,720 floats). */
#define CC1D_NOALLOC_WORKSPACE_FLOATS ((int64_t)1 << 21)

/*
 * Forward: out[b,c,t] = act(bias[c] + sum_k weight[c,k] * xx(b,c,t+k-(W-1)))
 * with xx(s) = x[b,c,s] for s >= 0, initial_states[b,c,s+W-1] for s < 0 when
 * given, else 0. With seq_idx, tap k is kept only when
 * seq_idx[b,s] == seq_idx[b,t], and positions with seq_idx[b,t] < 0 output 0.
 * final_states_out (optional) receives x[b,c,L-(W-1)+i], zero for indices
 * before 0 (initial_states is not used for it).
 * Semantics: src/causal_conv1d_mojo/fwd_cpu/kernel.mojo:61-119 and
 * src/causal_conv1d_mojo/_fn.py:31-50.
 */
typedef struct cc1d_fwd_params {
    const void* x;                 /* (batch, dim, seqlen) */
    const void* weight;            /* (dim, width) */
    const void* bias;              /* (dim,) or NULL */
    const int32_t* seq_idx;        /* (batch, seqlen) or NULL */
    const void* initial_states;    /* (batch, dim, width-1) or NULL */
    void* out;                     /* (batch, dim, seqlen) */
    void* final_states_out;        /* (batch, dim, width-1) or NULL */
    int64_t batch, dim, seqlen, width;
    int64_t x_stride[3];
    int64_t weight_stride[2];
    int64_t bias_stride;
    int64_t seq_idx_stride[2];
    int64_t initial_states_stride[3];
    int64_t out_stride[3];
    int64_t final_states_stride[3];
    int32_t dtype;                 /* enum cc1d_dtype, shared by every float tensor */
    int32_t apply_silu;            /* nonzero: SiLU (= swish) epilogue */
} cc1d_fwd_params;

/*
 * Fused backward: recomputes pre, dpre = dout * silu'(pre) (or dout), and
 * writes dx, dinitial_states (when initial_states is given) and ADDS the fp32
 * partial sums into dweight_acc (dim, width) and dbias_acc (dim,) -- the
 * caller zeroes them first, as in the reference (bwd_full/launch.mojo:10-12).
 * When dfinal_states is given, dx[..., L-m:] becomes
 * round(round(dx) + dfinal_states[..., W-1-m:]) with m = min(W-1, L), which is
 * the reference's separate in-dtype tail add (src/causal_conv1d_mojo/_fn.py:308-315).
 * Semantics: src/causal_conv1d_mojo/bwd_full_cpu/kernel.mojo:25-314.
 */
typedef struct cc1d_bwd_params {
    const void* x;
    const void* weight;
    const void* bias;              /* or NULL */
    const void* dout;
    const int32_t* seq_idx;        /* or NULL */
    const void* initial_states;    /* or NULL */
    const void* dfinal_states;     /* (batch, dim, width-1) or NULL */
    void* dx;
    float* dweight_acc;            /* (dim, width) fp32, accumulated into */
    float* dbias_acc;              /* (dim,) fp32 or NULL */
    void* dinitial_states;         /* required when initial_states is given; NULL with seq_idx */
    int64_t batch, dim, seqlen, width;
    int64_t x_stride[3];
    int64_t weight_stride[2];
    int64_t bias_stride;
    int64_t dout_stride[3];
    int64_t seq_idx_stride[2];
    int64_t initial_states_stride[3];
    int64_t dfinal_states_stride[3];
    int64_t dx_stride[3];
    int64_t dweight_acc_stride[2];
    int64_t dbias_acc_stride;
    int64_t dinitial_states_stride[3];
    int32_t dtype;
    int32_t apply_silu;
} cc1d_bwd_params;

/*
 * Weight/bias gradients in the dtype for cc1d_bwd_typed. The backward kernel
 * writes fp32 partial sums to `workspace` (no atomics, nothing to zero
 * first); a second kernel sums each channel's partials in a fixed order and
 * writes dweight (and dbias) rounded once to the dtype, so the result is the
 * same on every run.
 */
typedef struct cc1d_bwd_grads {
    void* dweight;                 /* (dim, width), dtype of the call */
    void* dbias;                   /* (dim,) or NULL */
    float* workspace;              /* at least cc1d_bwd_workspace_floats() floats */
    int64_t dweight_stride[2];
    int64_t dbias_stride;
    int64_t workspace_floats;      /* capacity of workspace */
} cc1d_bwd_grads;

/*
 * Decode update. x holds `seqlen` new tokens per (batch, channel). Linear
 * mode (cache_seqlens == NULL): the state row becomes the last state_len
 * values of cat(state, x). Circular mode: x[i] is written at
 * (cache_seqlens[b] + i) mod state_len (floored modulo) and the W-1 history
 * values are read just before that write head. conv_state_indices (optional)
 * redirects batch b to row conv_state_indices[b] of a state pool of
 * `state_rows` rows; an index < 0 (padding) or >= state_rows zeroes out[b]
 * and leaves the pool untouched. cache_seqlens is indexed by b.
 * Semantics: src/causal_conv1d_mojo/update_cpu/kernel.mojo:49-141.
 */
typedef struct cc1d_update_params {
    const void* x;                 /* (batch, dim, seqlen) */
    const void* weight;            /* (dim, width) */
    const void* bias;              /* (dim,) or NULL */
    void* conv_state;              /* (state_rows, dim, state_len), mutated */
    const int32_t* conv_state_indices; /* (batch,) contiguous or NULL */
    const int32_t* cache_seqlens;  /* (batch,) contiguous or NULL */
    void* out;                     /* (batch, dim, seqlen) */
    int64_t batch, dim, seqlen, width, state_len, state_rows;
    int64_t x_stride[3];
    int64_t weight_stride[2];
    int64_t bias_stride;
    int64_t conv_state_stride[3];
    int64_t out_stride[3];
    int32_t dtype;
    int32_t apply_silu;
} cc1d_update_params;

/*
 * Varlen state gather: states[i, :, state_len-n+j] = x[start+j, :] for the
 * last n = min(state_len, len_i) tokens of packed sequence i
 * (cu_seqlens[i] .. cu_seqlens[i+1]); all other entries are written 0 (all
 * bits clear). cu_seqlens values are clamped to [0, total_tokens]. It is a
 * copy, so any element type works: elem_bytes = 1, 2, 4, 8 or 16 moves
 * elements of that size bit for bit (fp64, integers, bool, complex ...) and
 * dtype is ignored; elem_bytes = 0 takes the size of dtype.
 * Semantics: src/causal_conv1d_mojo/causal_conv1d_varlen.py:29-61 (a torch
 * copy there, so dtype-agnostic).
 */
typedef struct cc1d_varlen_params {
    const void* x;                 /* (total_tokens, dim) */
    const int32_t* cu_seqlens;     /* (batch + 1,) contiguous */
    void* states;                  /* (batch, dim, state_len) */
    int64_t total_tokens, dim, batch, state_len;
    int64_t x_stride[2];
    int64_t states_stride[3];
    int32_t dtype;                 /* enum cc1d_dtype; used only when elem_bytes == 0 */
    int32_t elem_bytes;            /* 0, or 1 / 2 / 4 / 8 / 16 */
} cc1d_varlen_params;

int cc1d_abi_version(void);
const char* cc1d_strerror(int status);

int cc1d_fwd(const cc1d_fwd_params* params, void* stream);
int cc1d_bwd(const cc1d_bwd_params* params, void* stream);

/*
 * Backward with typed weight/bias gradients (what causal_conv1d_fn's
 * autograd backward returns, src/causal_conv1d_mojo/_fn.py:258-332): dx,
 * dinitial_states and the dfinal_states tail as in cc1d_bwd, and
 * dweight/dbias written through `grads` instead of accumulated into
 * params->dweight_acc / dbias_acc (ignored here). Two kernels; no fill.
 * cc1d_bwd_workspace_floats returns the workspace size for these params
 * (< 0 for an invalid dtype or width).
 */
int64_t cc1d_bwd_workspace_floats(const cc1d_bwd_params* params);
int cc1d_bwd_typed(const cc1d_bwd_params* params, const cc1d_bwd_grads* grads, void* stream);

/*
 * cc1d_bwd_typed without a caller-provided workspace. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The
 * fp32 partial sums go to a static device array of
 * CC1D_NOALLOC_WORKSPACE_FLOATS floats inside the library (one per GPU,
 * held until the process ends); grads->workspace and
 * grads->workspace_floats are ignored. A problem whose
 * cc1d_bwd_workspace_floats() exceeds that size returns
 * CC1D_ERR_SCRATCH_LIMIT and enqueues nothing. The call allocates nothing;
 * its first call on a device looks up that device's copy of the array
 * (hipGetSymbolAddress), so make that first call outside graph capture.
 * Every call on one GPU shares the array: calls that overlap on one GPU (on
 * other streams or threads) race; calls ordered on one stream do not. The
 * results are those of cc1d_bwd_typed, bit for bit.
 */
int cc1d_bwd_typed_noalloc(const cc1d_bwd_params* params, const cc1d_bwd_grads* grads, void* stream);
int cc1d_update(const cc1d_update_params* params, void* stream);
int cc1d_varlen_states(const cc1d_varlen_params* params, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CC1D_H */
