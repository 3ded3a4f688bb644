// cc1d_varlen.hip -- packed-sequence state gather and small fill kernels.
//
// states[i, c, s] = x[end_i - (S - s), c] when that token belongs to sequence
// i (cu_seqlens[i] <= token < cu_seqlens[i+1]), else 0 -- the last
// state_len tokens of each sequence, left zero-padded
// (src/causal_conv1d_mojo/causal_conv1d_varlen.py:29-61), for elements of
// 1, 2, 4, 8 or 16 bytes copied bit for bit. One thread per
// output element, channels fastest, so both the reads of x (token-major) and
// the writes of the (batch, state_len, dim)-allocated output are coalesced.
#include "cc1d_internal.hpp"

namespace cc1d {

struct VarArgs {
    cc1d_varlen_params p;
    int64_t n_items;
};

__device__ __forceinline__ int64_t clamp_tok(int64_t v, int64_t n) { return v < 0 ? 0 : (v > n ? n : v); }

// Elements are moved as raw bits of their size (E bytes), so any dtype works.
template <int E> struct Raw;
template <> struct Raw<1> { typedef uint8_t type; };
template <> struct Raw<2> { typedef uint16_t type; };
template <> struct Raw<4> { typedef uint32_t type; };
template <> struct Raw<8> { typedef uint64_t type; };
template <> struct Raw<16> { typedef u32x4 type; };

template <int E>
__global__ void __launch_bounds__(256) varlen_states_kernel(const VarArgs a) {
    typedef typename Raw<E>::type T;
    const cc1d_varlen_params& p = a.p;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n_items) return;
    const int64_t c = idx % p.dim;
    const int64_t rest = idx / p.dim;
    const int64_t s = rest % p.state_len;
    const int64_t i = rest / p.state_len;
    const int64_t end = clamp_tok(p.cu_seqlens[i + 1], p.total_tokens);
    int64_t start = clamp_tok(p.cu_seqlens[i], p.total_tokens);
    if (start < end - p.state_len) start = end - p.state_len;
    const int64_t n = end > start ? end - start : 0;
    const int64_t j = s - (p.state_len - n);  // index into the kept tokens
    T val{};
    if (j >= 0) val = static_cast<const T*>(p.x)[(start + j) * p.x_stride[0] + c * p.x_stride[1]];
    static_cast<T*>(p.states)[i * p.states_stride[0] + c * p.states_stride[1] + s * p.states_stride[2]] = val;
}

int varlen_elem_bytes(const cc1d_varlen_params& p) {
    if (p.elem_bytes != 0) return p.elem_bytes;
    return p.dtype == CC1D_DTYPE_FP32 ? 4 : 2;
}

int launch_varlen_states(const cc1d_varlen_params& p, hipStream_t stream) {
    VarArgs a;
    a.p = p;
    a.n_items = p.batch * p.state_len * p.dim;
    const dim3 grid((unsigned)ceil_div(a.n_items, 256));
    switch (varlen_elem_bytes(p)) {
    case 1: return launch(varlen_states_kernel<1>, grid, dim3(256), stream, a);
    case 2: return launch(varlen_states_kernel<2>, grid, dim3(256), stream, a);
    case 4: return launch(varlen_states_kernel<4>, grid, dim3(256), stream, a);
    case 8: return launch(varlen_states_kernel<8>, grid, dim3(256), stream, a);
    case 16: return launch(varlen_states_kernel<16>, grid, dim3(256), stream, a);
    default: return CC1D_ERR_DTYPE;
    }
}

template <typename U>
__global__ void __launch_bounds__(256) zero3_kernel(U* ptr, int64_t n0, int64_t n1, int64_t n2, int64_t s0,
                                                    int64_t s1, int64_t s2) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n0 * n1 * n2) return;
    const int64_t i2 = idx % n2;
    const int64_t r = idx / n2;
    const int64_t i1 = r % n1;
    const int64_t i0 = r / n1;
    ptr[i0 * s0 + i1 * s1 + i2 * s2] = U{};
}

int launch_zero3(void* ptr, int esize, int64_t n0, int64_t n1, int64_t n2, const int64_t* stride,
                 hipStream_t stream) {
    const int64_t n = n0 * n1 * n2;
    if (n == 0) return CC1D_OK;
    const dim3 grid((unsigned)ceil_div(n, 256));
    if (esize == 2)
        return launch(zero3_kernel<uint16_t>, grid, dim3(256), stream, static_cast<uint16_t*>(ptr), n0, n1, n2,
                      stride[0], stride[1], stride[2]);
    return launch(zero3_kernel<uint32_t>, grid, dim3(256), stream, static_cast<uint32_t*>(ptr), n0, n1, n2,
                  stride[0], stride[1], stride[2]);
}

}  // namespace cc1d
