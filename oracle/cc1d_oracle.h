/*
 * cc1d_oracle.h -- CPU restatement of the reference's CPU path for the
 * depthwise causal conv1d (forward, fused backward, decode update, varlen
 * state gather).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / CPU baseline. The product (causal_conv1d_amd) never calls it.
 *
 * The argument lists mirror the flat runtime tuples the reference's CPU
 * wrappers pass to their kernels:
 *   fwd    : src/causal_conv1d_mojo/fwd_cpu/__init__.py:139-170
 *   bwd    : src/causal_conv1d_mojo/bwd_full_cpu/__init__.py:338-379
 *   update : src/causal_conv1d_mojo/update_cpu/__init__.py:162-193
 * Strides are in elements. Absent optional tensors are NULL pointers.
 * dtype codes follow src/causal_conv1d_mojo/_dtype.py:16-20
 * (0 = fp16, 1 = bf16, 2 = fp32).
 */
#ifndef CC1D_ORACLE_H
#define CC1D_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Returns 0 on success, nonzero on a bad argument. */
int oracle_fwd(int dtype, int width, int apply_silu,
               const void* x, const void* weight, const void* bias, void* out,
               int64_t batch, int64_t dim, int64_t seqlen,
               int64_t x_s0, int64_t x_s1, int64_t x_s2,
               int64_t w_s0, int64_t w_s1,
               int64_t o_s0, int64_t o_s1, int64_t o_s2,
               const int32_t* seq_idx, int64_t si_s0, int64_t si_s1,
               const void* init, int64_t is_s0, int64_t is_s1, int64_t is_s2);

/* dweight_acc (dim, width) and dbias_acc (dim,) are fp32, contiguous, and
 * are ADDED to (callers pass zeros), as in the reference. */
int oracle_bwd(int dtype, int width, int apply_silu,
               const void* x, const void* weight, const void* bias,
               const void* dout, void* dx, float* dweight_acc, float* dbias_acc,
               int64_t batch, int64_t dim, int64_t seqlen,
               int64_t x_s0, int64_t x_s1, int64_t x_s2,
               int64_t w_s0, int64_t w_s1,
               int64_t g_s0, int64_t g_s1, int64_t g_s2,
               int64_t dx_s0, int64_t dx_s1, int64_t dx_s2,
               const int32_t* seq_idx, int64_t si_s0, int64_t si_s1,
               const void* init, int64_t is_s0, int64_t is_s1, int64_t is_s2,
               void* dinit, int64_t di_s0, int64_t di_s1, int64_t di_s2);

/* state_indices / cache_seqlens are contiguous int32 (batch,) or NULL. */
int oracle_update(int dtype, int width, int apply_silu,
                  const void* x, const void* weight, const void* bias,
                  void* conv_state, void* out,
                  int64_t batch, int64_t dim, int64_t seqlen, int64_t state_len,
                  int64_t x_s0, int64_t x_s1, int64_t x_s2,
                  int64_t w_s0, int64_t w_s1,
                  int64_t cs_s0, int64_t cs_s1, int64_t cs_s2,
                  int64_t o_s0, int64_t o_s1, int64_t o_s2,
                  const int32_t* state_indices, const int32_t* cache_seqlens);

/* Scalar conversions exposed so tests can pin them against torch. */
float oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
int oracle_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* CC1D_ORACLE_H */
