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
//                    Ragged rows (a start that is not 16-byte aligned, or a
//                    length that is not a multiple of the vector) are read in
//                    the 16-byte vectors of their own memory: a row that starts
//                    m elements past a vector boundary is walked from that
//                    boundary, its first m elements (the previous row's) are
//                    replaced by initial_states or zero, and the vectors it
//                    shares with its neighbours are stored element by element.
//   fwd_cl        -- rows contiguous along channels (channel-last). A lane owns
//                    4 bytes of adjacent channels, a wavefront a tile of 16
//                    time steps (plus W-1 halo rows) of 64 lanes' channels,
//                    all loaded before any arithmetic; seq_idx is
//                    wave-uniform here.
//   fwd_generic   -- any strides / alignment; one thread per
//                    (b, c, chunk of time), lanes on adjacent channels.
#include "cc1d_internal.hpp"

namespace cc1d {

struct FwdArgs {
    cc1d_fwd_params p;
    int32_t ragged;    // rows_vec: rows may start off a 16-byte boundary / end inside a vector (kernel variant)
    FastDiv nseg_div;  // rows_vec: item -> row
    FastDiv dim_div;   // rows_vec: row -> batch entry
    int64_t nseg;     // segments (rows_vec), tiles (cl) or chunks (generic) per row
    int64_t n_items;  // work items: segments / tiles / threads
    int64_t chunk;    // time steps per item (cl / generic)
    int64_t ngroups;  // channel groups (cl)
};

// One wavefront-segment of one row. FULL: the whole segment lies inside the
// row (no per-vector bounds checks).
//
// Positions t here count from the 16-byte boundary at or before the row's
// first element: the row holds t in [m, m + L) (m = 0 for an aligned row), so
// every vector access is aligned. A 16-byte vector that holds one of the
// row's elements lies in the same memory page, so reading it whole is safe.
template <typename T, int W, int VPT, bool SILU, bool SEQ, bool FULL, bool RAG>
__device__ __forceinline__ void fwd_rows_segment(const cc1d_fwd_params& p, int lane, int64_t b, int64_t c,
                                                 int32_t t0, int32_t m) {
    constexpr int EPV = elems16<T>::value;
    constexpr int H = W - 1;
    const int32_t L = (int32_t)p.seqlen;
    const int32_t Lv = L + m;  // end of the row
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1] - m;
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1] - m;

    u32x4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        v[j] = (FULL || t < Lv) ? vload_nt(xr + t) : vzero();
    }
    u32x4 h = vzero();
    if (lane == 0 && t0 > 0) h = vload(xr - EPV + t0);

    int32_t id[VPT][EPV];
    int32_t hid[H];
    if constexpr (SEQ) {
        const int32_t* __restrict__ sr = p.seq_idx + b * p.seq_idx_stride[0];  // unit time stride
        // ragged rows: a vector's ids start rid ids past a 16-byte boundary
        // (its first position, t - m, is a multiple of 4 plus -m); the row's
        // first id a0 past one
        const int a0 = RAG ? (int)uniform32((uint32_t)(reinterpret_cast<uintptr_t>(sr) / 4) & 3u) : 0;
        const int rid = (a0 - m) & 3;
        IdsRaw<EPV> raw[RAG ? VPT : 1];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int32_t t = t0 + (j * 64 + lane) * EPV;
            if constexpr (!RAG) {  // aligned rows: 16-byte vectors of 4 ids
#pragma unroll
                for (int q = 0; q < EPV / 4; ++q) {
                    const u32x4 s = (FULL || t < L) ? *reinterpret_cast<const u32x4*>(sr + t + 4 * q)
                                                    : u32x4{0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
#pragma unroll
                    for (int r = 0; r < 4; ++r) id[j][4 * q + r] = (int32_t)s[r];
                }
            } else {
                ids_load<EPV, !FULL>(sr, L, t - m, rid, a0, raw[j]);
            }
        }
        if constexpr (RAG) {  // -1 outside the row
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const int32_t pos = t0 + (j * 64 + lane) * EPV - m;
                const int32_t vs = t0 + j * 64 * EPV;  // vector j of lane 0: inside the row in every lane?
                if (FULL || (vs >= m && vs + 64 * EPV <= Lv)) ids_shift<EPV, false>(raw[j], L, pos, rid, id[j]);
                else ids_shift<EPV, true>(raw[j], L, pos, rid, id[j]);
            }
        }
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int32_t pos = t0 - H + i - m;
            hid[i] = (lane == 0 && pos >= 0) ? sr[pos] : -1;
        }
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
    // the row's first vector holds m elements of the previous row: they are
    // positions -m .. -1 of this one (initial_states or zero)
    if (RAG && !FULL && t0 == 0 && m > 0 && lane == 0) {
        float f[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e)  // initial_states slot e - m + H (none when negative)
            f[e] = e >= m ? vget<T>(v[0], e) : pick<H>(hinit, e - m + H);
        v[0] = vpack<T>(f);
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
        // before the row (t0 == 0, lane 0): position i - H - m, initial_states slot i - m
#pragma unroll
        for (int i = 0; i < H; ++i) {
            if constexpr (FULL || !RAG)  // m == 0 whenever a first segment is full
                win[i] = (j == 0 && use_init) ? hinit[i] : vget<T>(pv, EPV - H + i);
            else
                win[i] = (j == 0 && use_init) ? pick<H>(hinit, i - m) : vget<T>(pv, EPV - H + i);
        }
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
        if constexpr (!RAG) {
            if (FULL || t < L) vstore_nt(orow + t, vpack<T>(o));
        } else {
            const u32x4 ov = vpack<T>(o);
            if (FULL || (t >= m && t + EPV <= Lv)) {
                vstore_nt(orow + t, ov);
            } else if (t < Lv) {  // a vector shared with a neighbouring row
#pragma unroll
                for (int e = 0; e < EPV; ++e)
                    if ((uint32_t)(t + e - m) < (uint32_t)(Lv - m)) st_elem<T>(orow + t + e, ov, e);
            }
        }

        // final_states (_fn.py:31-50): the lane holding the row's last
        // position writes the last W-1 columns from its window (they are
        // positions t - H .. t + EPV - 1)
        if (p.final_states_out != nullptr && (RAG ? (t < Lv && Lv <= t + EPV) : t + EPV == L)) {
            T* fs = static_cast<T*>(p.final_states_out) + b * p.final_states_stride[0] +
                    c * p.final_states_stride[1];
#pragma unroll
            for (int i = 0; i < H; ++i) {  // position L - H + i is window slot Lv + i - t
                const float fv = RAG ? pick<H + EPV>(win, Lv + i - t) : win[EPV + i];  // aligned: t + EPV == L
                st(fs, i * p.final_states_stride[2], (L - H + i >= 0) ? fv : 0.0f);
            }
        }
    }
}

// Item = (row, segment) with row = b * dim + c; four wavefronts per block take
// four consecutive items, i.e. adjacent segments of a row or adjacent rows.
// All index arithmetic is 32-bit (the launcher checks the ranges).
template <typename T, int W, int VPT, bool SILU, bool SEQ, bool RAG>
__global__ void __launch_bounds__(256) fwd_rows_vec(const FwdArgs a) {
    constexpr int SEG = 64 * VPT * elems16<T>::value;
    const cc1d_fwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const uint32_t item = uniform32(blockIdx.x * 4u + (threadIdx.x >> 6));
    if (item >= (uint32_t)a.n_items) return;
    // (row, segment) and (b, c) by the host's invariant-divisor constants
    const uint32_t row = a.nseg_div.div(item);
    const int32_t t0 = (int32_t)((item - row * (uint32_t)a.nseg) * SEG);
    const uint32_t b = a.dim_div.div(row);
    const uint32_t c = row - b * (uint32_t)p.dim;
    constexpr int EPV = elems16<T>::value;
    // ragged rows: the row starts m elements past a 16-byte boundary
    int32_t m = 0;
    if constexpr (RAG) {
        const T* xrow = static_cast<const T*>(p.x) + (int64_t)b * p.x_stride[0] + (int64_t)c * p.x_stride[1];
        m = (int32_t)uniform32((uint32_t)(reinterpret_cast<uintptr_t>(xrow) / sizeof(T)) & (EPV - 1));
    }
    const int32_t Lv = (int32_t)p.seqlen + m;
    if (RAG && t0 >= Lv) return;  // the row ends before this segment
    if ((t0 > 0 || m == 0) && t0 + SEG <= Lv)
        fwd_rows_segment<T, W, VPT, SILU, SEQ, true, RAG>(p, lane, b, c, t0, m);
    else
        fwd_rows_segment<T, W, VPT, SILU, SEQ, false, RAG>(p, lane, b, c, t0, m);
}

// Channel-last (unit channel stride), tiled: a lane owns CPL adjacent
// channels (one CPL-element vector per time step); a wavefront covers
// 64 * CPL channels of a tile of TS time steps and issues the loads of all
// TS + W - 1 rows of its window (the W-1 halo rows before the tile included)
// before any arithmetic. seq_idx is one value per time step, the same for
// every lane: it is read through the scalar cache, and a tile whose window
// holds one sequence id (>= 0) takes the ungated path. Item order: channel
// group fastest, then tile, then batch. Index arithmetic is 32-bit inside a
// batch (the launcher checks the ranges).
template <typename T, int W, int CPL, int TS, bool SILU, bool SEQ>
__global__ void __launch_bounds__(256) fwd_cl(const FwdArgs a) {
    constexpr int H = W - 1;
    constexpr int NR = TS + H;
    using V = Lanes<T, CPL>;
    const cc1d_fwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const uint32_t item = uniform32(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (item >= (uint32_t)a.n_items) return;
    const uint32_t ngroups = (uint32_t)a.ngroups, ntiles = (uint32_t)a.nseg;
    const uint32_t g = item % ngroups;
    const uint32_t rest = item / ngroups;
    const uint32_t tile = rest % ntiles;
    const uint32_t b = rest / ntiles;
    const int32_t L = (int32_t)p.seqlen;
    const int32_t c0 = (int32_t)((g * 64 + lane) * CPL);
    const bool active = c0 < (int32_t)p.dim;
    const int32_t t0 = (int32_t)(tile * TS);
    const int32_t xs2 = (int32_t)p.x_stride[2], os2 = (int32_t)p.out_stride[2];
    const T* __restrict__ xb = static_cast<const T*>(p.x) + b * p.x_stride[0] + c0;
    T* __restrict__ ob = static_cast<T*>(p.out) + b * p.out_stride[0] + c0;

    V xv[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int32_t s = t0 - H + i;
        xv[i].zero();
        if (active && s >= 0 && s < L) xv[i].template load<false>(xb + s * xs2);
    }
    if (p.initial_states != nullptr && t0 < H && active) {
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int32_t s = t0 - H + i;
            if (s < 0) {
                float f[CPL];
#pragma unroll
                for (int e = 0; e < CPL; ++e)
                    f[e] = ld(static_cast<const T*>(p.initial_states),
                              b * p.initial_states_stride[0] + (c0 + e) * p.initial_states_stride[1] +
                                  (s + H) * p.initial_states_stride[2]);
                xv[i].set(f);
            }
        }
    }

    float w[W][CPL], bias[CPL];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
        const int64_t c = active ? c0 + e : 0;
#pragma unroll
        for (int k = 0; k < W; ++k)
            w[k][e] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
        bias[e] = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;
    }

    int32_t id[NR];
    bool one_id = true;
    if constexpr (SEQ) {
        // lane i < NR reads the id of position t0 - H + i (clamped address,
        // -1 outside the row); the window's ids then reach every lane through
        // readlane, with no dependent scalar reads.
        static_assert(NR <= 64, "the id window must fit in one wavefront");
        const int32_t* sr = p.seq_idx + b * p.seq_idx_stride[0];
        const int32_t s = t0 - H + lane;
        int32_t lid = sr[(s < 0 ? 0 : (s < L ? s : L - 1)) * (int32_t)p.seq_idx_stride[1]];
        if (s < 0 || s >= L) lid = -1;
        const int32_t id_cur = __builtin_amdgcn_readlane(lid, H);
        // rows outside [0, L) hold zeros (seq_idx excludes initial_states) or
        // feed outputs that are not stored, so they do not break a single-id window
        one_id = id_cur >= 0 && __ballot(lane < NR && s >= 0 && s < L && lid != id_cur) == 0;
#pragma unroll
        for (int i = 0; i < NR; ++i) id[i] = __builtin_amdgcn_readlane(lid, i);
    }

    auto emit = [&](auto gated) {
        constexpr bool G = decltype(gated)::value;
#pragma unroll
        for (int u = 0; u < TS; ++u) {
            const int32_t t = t0 + u;
            float o[CPL];
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                float col[W], wc[W];
#pragma unroll
                for (int k = 0; k < W; ++k) {
                    col[k] = xv[u + k].get(e);
                    wc[k] = w[k][e];
                }
                float acc;
                if constexpr (G) acc = conv_taps_gated<W>(bias[e], wc, col, id + u);
                else acc = conv_taps<W>(bias[e], wc, col);
                if constexpr (SILU) acc = silu(acc);
                if constexpr (G) {
                    if (id[u + H] < 0) acc = 0.0f;
                }
                o[e] = acc;
            }
            if (active && t < L) {
                V ov;
                ov.set(o);
                ov.template store<true>(ob + t * os2);
            }
        }
    };
    if (!SEQ || one_id) emit(std::false_type{});
    else if constexpr (SEQ) emit(std::true_type{});

    if (p.final_states_out != nullptr && active && t0 + TS >= L) {
        T* fs = static_cast<T*>(p.final_states_out) + b * p.final_states_stride[0];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int32_t r = L - t0 + i;  // register row of position L - H + i
            float f[CPL];
#pragma unroll
            for (int e = 0; e < CPL; ++e) f[e] = 0.0f;
#pragma unroll
            for (int q = 0; q < NR; ++q)
                if (q == r && L - H + i >= 0) {
#pragma unroll
                    for (int e = 0; e < CPL; ++e) f[e] = xv[q].get(e);
                }
#pragma unroll
            for (int e = 0; e < CPL; ++e)
                st(fs, (c0 + e) * p.final_states_stride[1] + i * p.final_states_stride[2], f[e]);
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

// channel-last launch shape: time steps per wavefront tile
constexpr int kClTS = 16;
constexpr int kClTSSmall = 8;  // on grids of fewer than 4096 wavefronts

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

// ragged rows (a seqlen that is not a multiple of the vector, or rows that do
// not start on a 16-byte boundary): unit time stride, and out laid out like x
// modulo the vector -- the same element strides modulo EPV and bases a
// multiple of 16 bytes apart -- so every row of out starts as far past a
// 16-byte boundary as its row of x; seq_idx with a unit time stride
template <typename T>
bool rows_ragged_ok(const cc1d_fwd_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    if (p.width - 1 > EPV) return false;
    if (p.x_stride[2] != 1 || p.out_stride[2] != 1) return false;
    if ((p.out_stride[0] - p.x_stride[0]) % EPV != 0 || (p.out_stride[1] - p.x_stride[1]) % EPV != 0) return false;
    if ((reinterpret_cast<intptr_t>(p.out) - reinterpret_cast<intptr_t>(p.x)) % 16 != 0) return false;
    if (p.seq_idx != nullptr && (p.seq_idx_stride[1] != 1 || reinterpret_cast<uintptr_t>(p.seq_idx) % 4 != 0))
        return false;
    const int64_t lim = (int64_t)1 << 31;
    if (p.seqlen + 64 * 4 * EPV + EPV >= lim) return false;
    if (p.batch * p.dim * ceil_div(p.seqlen + EPV, 64 * EPV) * 4 >= ((int64_t)1 << 32)) return false;
    return true;
}

// channel-last tiles: unit channel stride, CPL | dim, rows aligned to the
// CPL-channel lane vector, 32-bit positions inside a batch
template <typename T, int CPL>
bool cl_ok(const cc1d_fwd_params& p) {
    constexpr int64_t NB = CPL * (int64_t)sizeof(T);
    if (p.x_stride[1] != 1 || p.out_stride[1] != 1) return false;
    if (p.dim % CPL != 0) return false;
    if ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.out)) % NB) return false;
    if (p.x_stride[0] % CPL || p.x_stride[2] % CPL || p.out_stride[0] % CPL || p.out_stride[2] % CPL) return false;
    const int64_t span = p.seqlen + kClTS + 16;  // furthest row a tile touches
    const int64_t lim = (int64_t)1 << 31;
    if (p.dim >= lim || span * p.x_stride[2] >= lim || span * p.out_stride[2] >= lim) return false;
    if (p.seq_idx != nullptr && span * p.seq_idx_stride[1] >= lim) return false;
    if (p.batch * ceil_div(p.dim / CPL, 64) * ceil_div(p.seqlen, kClTS) >= lim * 2) return false;
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
                a.ragged = 0;
                const int64_t rows = p.batch * p.dim;
                if constexpr (W - 1 <= EPV) {
                    const bool aligned = rows_vec_ok<T>(p);
                    if (aligned || rows_ragged_ok<T>(p)) {
                        a.ragged = aligned ? 0 : 1;
                        // vectors a row spans: a ragged row may start up to EPV - 1
                        // elements past a vector boundary
                        const int64_t nvec = aligned ? p.seqlen / EPV : ceil_div(p.seqlen + EPV - 1, EPV);
                        const int64_t per = ceil_div(nvec, 64);
                        int vpt = per >= 4 ? 4 : (per >= 2 ? 2 : 1);
                        // ragged rows (measured at C2's batch and dim; aligned ones
                        // were faster without either): one segment of 4 vectors per
                        // lane instead of two of 2 with the same lane slots when the
                        // grid keeps 2048 wavefronts (L = 1031: 22.3 instead of
                        // 25.1 us), and 2 instead of 4 when a row a
                        // little longer than a multiple of the 4-vector segment would
                        // leave its last one mostly empty and 2 take at most 85 % of
                        // the lane slots (L = 2047: 34.2 instead of 37.6 us)
                        if (!aligned && per == 3 && rows >= 2048) vpt = 4;
                        else if (!aligned && vpt == 4 &&
                                 ceil_div(nvec, (int64_t)128) * 128 * 100 <= ceil_div(nvec, (int64_t)256) * 256 * 85)
                            vpt = 2;
                        // a grid of fewer than 2048 wavefronts (2 per SIMD): half the
                        // vectors per lane, twice the wavefronts (B = 1, D = 768,
                        // L = 2048: 3.03 instead of 3.41 us; D = 512, L = 1024:
                        // 2.40 instead of 2.53)
                        if (vpt == 4 && rows * ceil_div(nvec, (int64_t)256) < 2048) vpt = 2;
                        if (vpt == 2 && rows * ceil_div(nvec, (int64_t)128) < 2048) vpt = 1;
                        a.nseg = ceil_div(nvec, 64 * (int64_t)vpt);
                        a.n_items = rows * a.nseg;
                        a.nseg_div = FastDiv((uint32_t)a.nseg);
                        a.dim_div = FastDiv((uint32_t)p.dim);
                        const dim3 grid((unsigned)ceil_div(a.n_items, 4));
                        return with_flag(p.seq_idx != nullptr, [&](auto qc) {
                            constexpr bool SEQ = decltype(qc)::value;
                            return with_flag(a.ragged != 0, [&](auto rc) {
                                constexpr bool RAG = decltype(rc)::value;
                                if (vpt == 4) return launch(fwd_rows_vec<T, W, 4, SILU, SEQ, RAG>, grid, dim3(256), stream, a);
                                if (vpt == 2) return launch(fwd_rows_vec<T, W, 2, SILU, SEQ, RAG>, grid, dim3(256), stream, a);
                                return launch(fwd_rows_vec<T, W, 1, SILU, SEQ, RAG>, grid, dim3(256), stream, a);
                            });
                        });
                    }
                }
                constexpr int CPL = 4 / (int)sizeof(T);
                if (cl_ok<T, CPL>(p)) {
                    a.ngroups = ceil_div(p.dim / CPL, 64);
                    // 8-step tiles when 16-step ones would give fewer than 4096
                    // wavefronts: a tile is one round trip to memory, so a small
                    // grid gains from twice the wavefronts (bf16, B = 1, D = 768,
                    // L = 2048: 4.3 instead of 5.1 us; C3 keeps 16: 24.1 against 24.9)
                    a.chunk = p.batch * a.ngroups * ceil_div(p.seqlen, (int64_t)kClTS) < 4096 ? kClTSSmall : kClTS;
                    a.nseg = ceil_div(p.seqlen, a.chunk);
                    a.n_items = p.batch * a.nseg * a.ngroups;
                    const dim3 grid((unsigned)ceil_div(a.n_items, 4));
                    return with_flag(p.seq_idx != nullptr, [&](auto qc) {
                        constexpr bool SEQ = decltype(qc)::value;
                        if (a.chunk == kClTSSmall)
                            return launch(fwd_cl<T, W, CPL, kClTSSmall, SILU, SEQ>, grid, dim3(256), stream, a);
                        return launch(fwd_cl<T, W, CPL, kClTS, SILU, SEQ>, grid, dim3(256), stream, a);
                    });
                }
                a.chunk = 64;
                a.nseg = ceil_div(p.seqlen, a.chunk);
                a.n_items = rows * a.nseg;
                const dim3 grid((unsigned)ceil_div(a.n_items, 256));
                return launch(fwd_generic<T, W, SILU>, grid, dim3(256), stream, a);
            });
        });
    });
}

}  // namespace cc1d
