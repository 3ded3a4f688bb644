// cc1d_fwd.hip -- forward kernels for gfx950.
//
// Semantics (per batch b, channel c, position t; the CPU definition the
// reference tests against is src/causal_conv1d_mojo/fwd_cpu/kernel.mojo:61-119):
//   pre = bias[c]; for k in 0..W-1: pre += w[c,k] * xx(t + k - (W-1))   (fp32, in that order)
//   out = silu(pre) or pre; 0 where seq_idx[b,t] < 0
// where xx(s) = x[b,c,s] (s >= 0), initial_states[b,c,s+W-1] (s < 0, when
// given) or 0, and with seq_idx a tap is kept only if seq_idx[b,s] == seq_idx[b,t].
//
// Kernels
//   fwd_rows_vec  -- rows contiguous along t (channel-first). One wavefront
//                    owns a segment of 64*VPT*EPV positions of one row; lane l
//                    holds 16-byte vectors l, l+64, ... of the segment, so each
//                    load instruction covers 1 KB of contiguous HBM. The (W-1)
//                    halo before a vector comes from the neighbouring lane
//                    (ds_bpermute); only lane 0 of a segment reads one extra
//                    vector from global memory. No LDS, no barriers.
//   fwd_cols_vec  -- rows contiguous along channels (channel-last). A lane owns
//                    EPV adjacent channels (one 16-byte vector per time step)
//                    and walks a tile of time steps with a register window of
//                    the previous W-1 steps; seq_idx is wave-uniform here.
//   fwd_generic   -- any strides / alignment; one thread per
//                    (b, c, chunk of time), lanes on adjacent channels.
#include "cc1d_internal.hpp"

namespace cc1d {

struct FwdArgs {
    cc1d_fwd_params p;
    int64_t nseg;     // segments (vec) or chunks (generic) per row
    int64_t n_items;  // work items: segments / tiles / threads
    int64_t chunk;    // time steps per item (generic / cols)
    int64_t ngroups;  // channel groups (cols)
};

// One wavefront-segment of one row. FULL: the whole segment lies inside the
// row (no per-vector bounds checks).
template <typename T, int W, int VPT, bool SILU, bool SEQ, bool FULL>
__device__ __forceinline__ void fwd_rows_segment(const cc1d_fwd_params& p, int lane, int64_t b, int64_t c,
                                                 int32_t t0) {
    constexpr int EPV = elems16<T>::value;
    constexpr int H = W - 1;
    const int32_t L = (int32_t)p.seqlen;
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];

    u32x4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        v[j] = (FULL || t < L) ? vload_nt(xr + t) : vzero();
    }
    u32x4 h = vzero();
    if (lane == 0 && t0 > 0) h = vload(xr - EPV + t0);

    int32_t id[VPT][EPV];
    int32_t hid[H];
    if constexpr (SEQ) {
        const int32_t* __restrict__ sr = p.seq_idx + b * p.seq_idx_stride[0];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int32_t t = t0 + (j * 64 + lane) * EPV;
#pragma unroll
            for (int q = 0; q < EPV / 4; ++q) {
                const u32x4 s = (FULL || t < L) ? *reinterpret_cast<const u32x4*>(sr + t + 4 * q)
                                                : u32x4{0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
#pragma unroll
                for (int r = 0; r < 4; ++r) id[j][4 * q + r] = (int32_t)s[r];
            }
        }
#pragma unroll
        for (int i = 0; i < H; ++i)
            hid[i] = (lane == 0 && t0 - H + i >= 0) ? sr[t0 - H + i] : -1;
    }

    float w[W];
    const T* __restrict__ wr = static_cast<const T*>(p.weight) + c * p.weight_stride[0];
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = ld(wr, k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;

    const bool use_init = p.initial_states != nullptr && t0 == 0 && lane == 0;
    float hinit[H];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        hinit[i] = 0.0f;
        if (use_init)
            hinit[i] = ld(static_cast<const T*>(p.initial_states),
                          b * p.initial_states_stride[0] + c * p.initial_states_stride[1] +
                              i * p.initial_states_stride[2]);
    }

    constexpr int D0 = ((EPV - H) * (int)sizeof(T)) / 4;  // first dword of the needed tail
    const int prev_lane = (lane + 63) & 63;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        u32x4 pv = vzero();
#pragma unroll
        for (int d = D0; d < 4; ++d) {
            const uint32_t send = (lane == 63) ? (j > 0 ? v[j > 0 ? j - 1 : 0][d] : 0u) : v[j][d];
            pv[d] = lane_get(send, prev_lane);
        }
        if (j == 0 && lane == 0) pv = h;
        float win[H + EPV];
#pragma unroll
        for (int i = 0; i < H; ++i) win[i] = (j == 0 && use_init) ? hinit[i] : vget<T>(pv, EPV - H + i);
#pragma unroll
        for (int i = 0; i < EPV; ++i) win[H + i] = vget<T>(v[j], i);

        int32_t sw[H + EPV];
        if constexpr (SEQ) {
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const int32_t send = (lane == 63) ? (j > 0 ? id[j > 0 ? j - 1 : 0][EPV - H + i] : -1)
                                                  : id[j][EPV - H + i];
                const int32_t r = lane_get(send, prev_lane);
                sw[i] = (j == 0 && lane == 0) ? hid[i] : r;
            }
#pragma unroll
            for (int i = 0; i < EPV; ++i) sw[H + i] = id[j][i];
        }

        float o[EPV];
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
            float acc;
            if constexpr (SEQ) acc = conv_taps_gated<W>(bias, w, win + i, sw + i);
            else acc = conv_taps<W>(bias, w, win + i);
            if constexpr (SILU) acc = silu(acc);
            if constexpr (SEQ) {
                if (sw[H + i] < 0) acc = 0.0f;
            }
            o[i] = acc;
        }
        if (FULL || t < L) vstore_nt(orow + t, vpack<T>(o));

        // final_states (_fn.py:31-50): the lane holding position L-1 owns the
        // last W-1 columns (L % EPV == 0 on this path, so they are win[EPV..]).
        if (p.final_states_out != nullptr && t + EPV == L) {
            T* fs = static_cast<T*>(p.final_states_out) + b * p.final_states_stride[0] +
                    c * p.final_states_stride[1];
#pragma unroll
            for (int i = 0; i < H; ++i)
                st(fs, i * p.final_states_stride[2], (L - H + i >= 0) ? win[EPV + i] : 0.0f);
        }
    }
}

// Item = (row, segment) with row = b * dim + c; four wavefronts per block take
// four consecutive items, i.e. adjacent segments of a row or adjacent rows.
// All index arithmetic is 32-bit (the launcher checks the ranges).
template <typename T, int W, int VPT, bool SILU, bool SEQ>
__global__ void __launch_bounds__(256) fwd_rows_vec(const FwdArgs a) {
    constexpr int SEG = 64 * VPT * elems16<T>::value;
    const cc1d_fwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const uint32_t item = uniform32(blockIdx.x * 4u + (threadIdx.x >> 6));
    if (item >= (uint32_t)a.n_items) return;
    const uint32_t nseg = (uint32_t)a.nseg;
    const uint32_t row = item / nseg;
    const int32_t t0 = (int32_t)((item - row * nseg) * SEG);
    const uint32_t dim = (uint32_t)p.dim;
    const uint32_t b = row / dim;
    const uint32_t c = row - b * dim;
    if (t0 + SEG <= (int32_t)p.seqlen) fwd_rows_segment<T, W, VPT, SILU, SEQ, true>(p, lane, b, c, t0);
    else fwd_rows_segment<T, W, VPT, SILU, SEQ, false>(p, lane, b, c, t0);
}

// Channel-last: x[b, c, t] at b*xs0 + c + t*xs2 (unit channel stride).
// Work item = (b, tile of `chunk` steps, group of 64*CPL channels), group
// fastest. A lane owns CPL adjacent channels (one CPL-element vector per
// time step) and walks its tile with a register window of the previous W-1
// steps; the U loads of a step group are issued before their arithmetic.
// seq_idx is one value per time step here, identical for every lane.
template <typename T, int W, int CPL, int U, bool SILU, bool SEQ>
__global__ void __launch_bounds__(256) fwd_cols_vec(const FwdArgs a) {
    constexpr int H = W - 1;
    using V = Lanes<T, CPL>;
    const cc1d_fwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const int64_t item = uniform((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6));
    if (item >= a.n_items) return;
    const int64_t g = item % a.ngroups;
    const int64_t rest = item / a.ngroups;
    const int64_t tile = rest % a.nseg;
    const int64_t b = rest / a.nseg;
    const int64_t c0 = (g * 64 + lane) * CPL;
    const bool active = c0 < p.dim;
    const int64_t L = p.seqlen;
    const int64_t t0 = tile * a.chunk;
    const int64_t t1 = (t0 + a.chunk < L) ? t0 + a.chunk : L;
    const int64_t xs2 = p.x_stride[2], os2 = p.out_stride[2];
    const T* __restrict__ xb = static_cast<const T*>(p.x) + b * p.x_stride[0] + c0;
    T* __restrict__ ob = static_cast<T*>(p.out) + b * p.out_stride[0] + c0;

    float w[W][CPL];
    float bias[CPL];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
        const int64_t c = active ? c0 + e : 0;
#pragma unroll
        for (int k = 0; k < W; ++k)
            w[k][e] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
        bias[e] = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;
    }

    // win[i][e] = xx(t - H + i) for channel c0+e
    float win[W][CPL];
    int32_t wid[W];
    const int32_t* __restrict__ sr = SEQ ? p.seq_idx + b * p.seq_idx_stride[0] : nullptr;
#pragma unroll
    for (int i = 0; i < H; ++i) {
        const int64_t s = t0 - H + i;
        V hv;
        hv.zero();
        if (active && s >= 0) hv.template load<false>(xb + s * xs2);
#pragma unroll
        for (int e = 0; e < CPL; ++e) win[i][e] = hv.get(e);
        if (s < 0 && p.initial_states != nullptr && active) {
#pragma unroll
            for (int e = 0; e < CPL; ++e)
                win[i][e] = ld(static_cast<const T*>(p.initial_states),
                               b * p.initial_states_stride[0] + (c0 + e) * p.initial_states_stride[1] +
                                   (s + H) * p.initial_states_stride[2]);
        }
        if constexpr (SEQ) wid[i] = (s >= 0) ? sr[s * p.seq_idx_stride[1]] : -1;
    }

    for (int64_t tb = t0; tb < t1; tb += U) {
        V xv[U];
        int32_t ids[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t t = tb + u;
            xv[u].zero();
            if (active && t < t1) xv[u].template load<true>(xb + t * xs2);
            if constexpr (SEQ) ids[u] = (t < t1) ? sr[t * p.seq_idx_stride[1]] : -1;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t t = tb + u;
#pragma unroll
            for (int e = 0; e < CPL; ++e) win[H][e] = xv[u].get(e);
            if constexpr (SEQ) wid[H] = ids[u];
            float o[CPL];
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                float col[W], wc[W];
#pragma unroll
                for (int k = 0; k < W; ++k) { col[k] = win[k][e]; wc[k] = w[k][e]; }
                float acc;
                if constexpr (SEQ) acc = conv_taps_gated<W>(bias[e], wc, col, wid);
                else acc = conv_taps<W>(bias[e], wc, col);
                if constexpr (SILU) acc = silu(acc);
                if constexpr (SEQ) {
                    if (wid[H] < 0) acc = 0.0f;
                }
                o[e] = acc;
            }
            if (active && t < t1) {
                V ov;
                ov.set(o);
                ov.template store<true>(ob + t * os2);
            }
#pragma unroll
            for (int i = 0; i < H; ++i) {
#pragma unroll
                for (int e = 0; e < CPL; ++e) win[i][e] = win[i + 1][e];
                if constexpr (SEQ) wid[i] = wid[i + 1];
            }
        }
    }

    if (p.final_states_out != nullptr && active && t1 == L) {
        T* fs = static_cast<T*>(p.final_states_out) + b * p.final_states_stride[0];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int64_t s = L - H + i;
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                const float val = (s >= 0) ? ld(xb, s * xs2 + e) : 0.0f;
                st(fs, (c0 + e) * p.final_states_stride[1] + i * p.final_states_stride[2], val);
            }
        }
    }
}

template <typename T, int W, bool SILU>
__global__ void __launch_bounds__(256) fwd_generic(const FwdArgs a) {
    constexpr int H = W - 1;
    const cc1d_fwd_params& p = a.p;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n_items) return;
    const int64_t c = idx % p.dim;
    const int64_t rest = idx / p.dim;
    const int64_t ch = rest % a.nseg;
    const int64_t b = rest / a.nseg;
    const int64_t L = p.seqlen;
    const int64_t t0 = ch * a.chunk;
    const int64_t t1 = (t0 + a.chunk < L) ? t0 + a.chunk : L;
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];
    const int64_t xs = p.x_stride[2];
    const int32_t* sr = p.seq_idx ? p.seq_idx + b * p.seq_idx_stride[0] : nullptr;

    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        w[k] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;

    float win[W];
    int32_t wid[W];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        const int64_t s = t0 - H + i;
        if (s >= 0) {
            win[i] = ld(xr, s * xs);
        } else if (p.initial_states != nullptr) {
            win[i] = ld(static_cast<const T*>(p.initial_states),
                        b * p.initial_states_stride[0] + c * p.initial_states_stride[1] +
                            (s + H) * p.initial_states_stride[2]);
        } else {
            win[i] = 0.0f;
        }
        wid[i] = (sr != nullptr && s >= 0) ? sr[s * p.seq_idx_stride[1]] : -1;
    }
    for (int64_t t = t0; t < t1; ++t) {
        win[H] = ld(xr, t * xs);
        float acc;
        if (sr != nullptr) {
            wid[H] = sr[t * p.seq_idx_stride[1]];
            acc = conv_taps_gated<W>(bias, w, win, wid);
            if (SILU) acc = silu(acc);
            if (wid[H] < 0) acc = 0.0f;
        } else {
            acc = conv_taps<W>(bias, w, win);
            if (SILU) acc = silu(acc);
        }
        st(orow, t * p.out_stride[2], acc);
#pragma unroll
        for (int i = 0; i < H; ++i) {
            win[i] = win[i + 1];
            wid[i] = wid[i + 1];
        }
    }
    if (p.final_states_out != nullptr && t1 == L) {
        T* fs = static_cast<T*>(p.final_states_out) + b * p.final_states_stride[0] + c * p.final_states_stride[1];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int64_t s = L - H + i;
            st(fs, i * p.final_states_stride[2], (s >= 0) ? ld(xr, s * xs) : 0.0f);
        }
    }
}

// ---- launch selection ------------------------------------------------------

namespace {

// channel-last launch shape: channels per lane, steps per tile, steps in flight
constexpr int kColsCPL = 4;
constexpr int64_t kColsChunk = 64;
constexpr int kColsU = 8;

template <typename T>
bool rows_vec_ok(const cc1d_fwd_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    if (p.width - 1 > EPV) return false;
    if (p.x_stride[2] != 1 || p.out_stride[2] != 1) return false;
    if (p.seqlen % EPV != 0) return false;
    if (!aligned16(p.x) || !aligned16(p.out)) return false;
    if (p.x_stride[0] % EPV || p.x_stride[1] % EPV || p.out_stride[0] % EPV || p.out_stride[1] % EPV) return false;
    if (p.seq_idx != nullptr &&
        (p.seq_idx_stride[1] != 1 || p.seq_idx_stride[0] % 4 != 0 || !aligned16(p.seq_idx)))
        return false;
    // 32-bit index arithmetic: positions, rows and items (4 per block) must fit
    if (p.seqlen + 64 * 4 * EPV >= ((int64_t)1 << 31)) return false;
    if (p.batch * p.dim * ceil_div(p.seqlen, 64 * EPV) * 4 >= ((int64_t)1 << 32)) return false;
    return true;
}

// channel-last with CPL-channel lanes: unit channel stride, CPL | dim and
// every row start aligned to CPL elements
template <typename T, int CPL>
bool cols_vec_ok(const cc1d_fwd_params& p) {
    constexpr int64_t NB = CPL * (int64_t)sizeof(T);
    if (p.x_stride[1] != 1 || p.out_stride[1] != 1) return false;
    if (p.dim % CPL != 0) return false;
    if ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.out)) % NB) return false;
    if (p.x_stride[0] % CPL || p.x_stride[2] % CPL || p.out_stride[0] % CPL || p.out_stride[2] % CPL) return false;
    return true;
}

}  // namespace

int launch_fwd(const cc1d_fwd_params& p, hipStream_t stream) {
    return with_dtype(p.dtype, [&](auto tag) {
        using T = decltype(tag);
        constexpr int64_t EPV = elems16<T>::value;
        return with_width(p.width, [&](auto wc) {
            constexpr int W = decltype(wc)::value;
            return with_flag(p.apply_silu != 0, [&](auto sc) {
                constexpr bool SILU = decltype(sc)::value;
                FwdArgs a;
                a.p = p;
                a.chunk = 0;
                a.ngroups = 0;
                const int64_t rows = p.batch * p.dim;
                if constexpr (W - 1 <= EPV) {
                    if (rows_vec_ok<T>(p)) {
                        const int64_t nvec = p.seqlen / EPV;
                        const int64_t per = ceil_div(nvec, 64);
                        const int vpt = per >= 4 ? 4 : (per >= 2 ? 2 : 1);
                        a.nseg = ceil_div(nvec, 64 * (int64_t)vpt);
                        a.n_items = rows * a.nseg;
                        const dim3 grid((unsigned)ceil_div(a.n_items, 4));
                        return with_flag(p.seq_idx != nullptr, [&](auto qc) {
                            constexpr bool SEQ = decltype(qc)::value;
                            if (vpt == 4) fwd_rows_vec<T, W, 4, SILU, SEQ><<<grid, 256, 0, stream>>>(a);
                            else if (vpt == 2) fwd_rows_vec<T, W, 2, SILU, SEQ><<<grid, 256, 0, stream>>>(a);
                            else fwd_rows_vec<T, W, 1, SILU, SEQ><<<grid, 256, 0, stream>>>(a);
                            return launch_status();
                        });
                    }
                }
                constexpr int CPL = kColsCPL;
                if (cols_vec_ok<T, CPL>(p)) {
                    a.ngroups = ceil_div(p.dim / CPL, 64);
                    a.chunk = kColsChunk;
                    a.nseg = ceil_div(p.seqlen, a.chunk);
                    a.n_items = p.batch * a.nseg * a.ngroups;
                    const dim3 grid((unsigned)ceil_div(a.n_items, 4));
                    return with_flag(p.seq_idx != nullptr, [&](auto qc) {
                        constexpr bool SEQ = decltype(qc)::value;
                        fwd_cols_vec<T, W, CPL, kColsU, SILU, SEQ><<<grid, 256, 0, stream>>>(a);
                        return launch_status();
                    });
                }
                a.chunk = 64;
                a.nseg = ceil_div(p.seqlen, a.chunk);
                a.n_items = rows * a.nseg;
                const dim3 grid((unsigned)ceil_div(a.n_items, 256));
                fwd_generic<T, W, SILU><<<grid, 256, 0, stream>>>(a);
                return launch_status();
            });
        });
    });
}

}  // namespace cc1d
