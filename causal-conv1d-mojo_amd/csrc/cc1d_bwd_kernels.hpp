// cc1d_bwd_kernels.hpp -- fused backward kernels for gfx950 and their launch
// planning, templated on the storage type. Each cc1d_bwd_<dtype>.hip
// instantiates them for one type (the types compile in parallel);
// cc1d_bwd.hip dispatches on the dtype code.
//
// Semantics (src/causal_conv1d_mojo/bwd_full_cpu/kernel.mojo:25-314):
//   dpre[t] = dout[t] * silu'(pre[t]) (or dout[t] without SiLU); 0 for t
//             outside [0, L) and where seq_idx[t] < 0; pre is recomputed
//             exactly as in the forward.
//   dx[t]   = sum_k w[W-1-k] * dpre[t+k], tap k kept when seq_idx[t+k] == seq_idx[t]
//   dw[k]  += sum_t dpre[t] * xx(t+k-(W-1)), same gate as the forward
//   db     += sum_t dpre[t]
//   dinit[i] = sum_{k<=i} w[k] * dpre[i-k]   (i < W-1)
// dweight/dbias are reduced in fp32: per lane, then across the wavefront
// (row kernels: DPP adds) or the block (channel-last: LDS).
// cc1d_bwd adds the sums into the caller's zeroed fp32 accumulators with
// atomics -- as in the reference, the order of those adds (over batches and
// segments) is not fixed. cc1d_bwd_typed writes them as partial records
// instead, and bwd_reduce adds each channel's records in a fixed order
// (several records in flight per wavefront) and rounds once to the dtype.
//
// Kernels
//   bwd_rows_vec -- channel-first rows, same lane layout and item order as
//                   fwd_rows_vec (one item per wavefront, 4 per block),
//                   ragged rows included: positions count from the 16-byte
//                   boundary at or before the row's first element (the row is
//                   [m, m + L)), dpre is zero outside the row, and the vectors
//                   shared with neighbouring rows are stored element by element.
//   bwd_clw      -- channel-last (unit channel stride); a lane owns 4 bytes of
//                   adjacent channels, a wavefront walks a run of time steps.
//   bwd_generic  -- any strides; one thread per (b, c, chunk of time).
#pragma once

#include "cc1d_internal.hpp"

namespace cc1d {

struct BwdArgs {
    cc1d_bwd_params p;
    FastDiv nseg_div;  // rows_vec: item -> row
    FastDiv dim_div;   // rows_vec: row -> batch entry
    float* part;      // non-null: write weight/bias-gradient partial sums here instead of atomics
    int64_t nseg;     // rows_vec: segments per row; cl: run groups per row; generic: chunks per row
    int64_t n_items;  // rows_vec: (row, segment) items; generic: threads
    int64_t chunk;    // cl: time steps per run; generic: time steps per thread
    int64_t groups;   // cl: channel groups of 64 * CPL
    int32_t ragged;   // rows_vec: rows may start off a 16-byte boundary / end inside a vector (kernel variant)
};

// channel-first rows: (row, segment) items per block, one per wavefront
constexpr int kRowsWPB = 4;
// channel-last walk: time steps per chunk, per wavefront run, runs per block
constexpr int kClG = 4;
constexpr int kClR = 128;      // run length, and the shorter ones for small grids
constexpr int kClRMid = 64;
constexpr int kClRShort = 16;
constexpr int kClWPB = 8;

// Registers of one wavefront-segment of a row: VPT 16-byte vectors of x and
// dout per lane, plus the wave-uniform halos (scalar registers): the vector
// of x before the segment (used by lane 0) and x and dout of the first vector
// after it (used by lane 63); zero past either end of the row.
template <int VPT> struct RowTile {
    u32x4 v[VPT], gv[VPT], h, xn, gn;
};

// Issue the loads of segment t0 of row (b, c). FULL: the whole segment lies
// inside the row.
template <typename T, int VPT, bool FULL>
__device__ __forceinline__ void bwd_rows_load(const cc1d_bwd_params& p, int lane, int64_t b, int64_t c, int32_t t0,
                                              int32_t m, RowTile<VPT>& r) {
    constexpr int EPV = elems16<T>::value;
    constexpr int SEG = 64 * VPT * EPV;
    const int32_t L = (int32_t)p.seqlen + m;  // the row's end (its start is m)
    const int32_t tn = t0 + SEG;  // first position of the next segment
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1] - m;
    const T* __restrict__ gr = static_cast<const T*>(p.dout) + b * p.dout_stride[0] + c * p.dout_stride[1] - m;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        r.v[j] = (FULL || t < L) ? vload_nt(xr + t) : vzero();
        r.gv[j] = (FULL || t < L) ? vload_nt(gr + t) : vzero();
    }
    // halo vectors: wave-uniform reads at clamped (always valid) addresses
    const u32x4 hv = vload_uniform(xr + (t0 > 0 ? t0 - EPV : 0));
    const int32_t tq = tn < L ? tn : t0;
    const u32x4 xv = vload_uniform(xr + tq), gq = vload_uniform(gr + tq);
    r.h = t0 > 0 ? hv : vzero();
    r.xn = tn < L ? xv : vzero();
    r.gn = tn < L ? gq : vzero();
}

// One wavefront-segment of row (b, c) from its loaded tile, without seq_idx
// (bwd_rows_compute_seq below has it): writes dx (and dinitial_states) and
// adds this segment's weight/bias-gradient partials into pw / pb. RAG: the
// row starts m elements past a 16-byte boundary (m is 0 otherwise).
template <typename T, int W, int VPT, bool SILU, bool FULL, bool RAG>
__device__ __forceinline__ void bwd_rows_compute(const cc1d_bwd_params& p, int lane, int64_t b, int64_t c,
                                                 int32_t t0, int32_t m, RowTile<VPT> r, const float* w,
                                                 const float* wq, float bq, float* pw, float& pb) {
    constexpr int EPV = elems16<T>::value;
    constexpr int H = W - 1;
    constexpr int SEG = 64 * VPT * EPV;
    static_assert(H <= EPV, "the halo must fit in one 16-byte vector");
    const int32_t L = (int32_t)p.seqlen + m;  // the row is [m, L) in this segment's positions
    {
        const int32_t tn = t0 + SEG;  // first position of the next segment
        T* __restrict__ dxr = static_cast<T*>(p.dx) + b * p.dx_stride[0] + c * p.dx_stride[1] - m;

        const bool init_row = p.initial_states != nullptr && t0 == 0;  // wave-uniform
        const bool use_init = init_row && lane == 0;
        float hinit[H];
#pragma unroll
        for (int i = 0; i < H; ++i) hinit[i] = 0.0f;
        if (init_row) {
            const T* is = static_cast<const T*>(p.initial_states) + b * p.initial_states_stride[0] +
                          c * p.initial_states_stride[1];
#pragma unroll
            for (int i = 0; i < H; ++i) hinit[i] = ld_uniform(is + i * p.initial_states_stride[2]);
        }
        // dfinal_states of this row when the segment holds one of the row's
        // last W-1 positions (wave-uniform; a ragged row's may span two
        // segments, an aligned row's lie in its last vector)
        float dfin[H];
#pragma unroll
        for (int i = 0; i < H; ++i) dfin[i] = 0.0f;
        const bool dfin_row = p.dfinal_states != nullptr && tn > L - H;
        if (dfin_row) {
            const T* dfs = static_cast<const T*>(p.dfinal_states) + b * p.dfinal_states_stride[0] +
                           c * p.dfinal_states_stride[1];
#pragma unroll
            for (int i = 0; i < H; ++i) dfin[i] = ld_uniform(dfs + i * p.dfinal_states_stride[2]);
        }
        // a ragged row's first vector holds m elements of the previous row:
        // they are positions -m .. -1 of this one (x: initial_states or zero;
        // dout: zero), merged in as raw bits
        if (RAG && !FULL && t0 == 0 && m > 0 && lane == 0) {
            constexpr int EPD = EPV / 4;  // elements per dword
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t ib = 0;
#pragma unroll
                for (int k = 0; k < EPD; ++k)
                    ib |= tbits<T>(pick<H>(hinit, d * EPD + k - m + H)) << (32 / EPD * k);
                const uint32_t keep = ~lead_mask<T>(d, m);
                r.v[0][d] = (r.v[0][d] & keep) | (ib & ~keep);
                r.gv[0][d] &= keep;
            }
        }
        const auto& v = r.v;
        const auto& gv = r.gv;
        const u32x4 h = r.h, xn = r.xn, gn = r.gn;

        // The vectors are processed in order: dpre of vector j (with its
        // gradient partials), then dx of vector j - 1, which needs dpre of
        // vector j only for lane 63's last H positions (lane 0's first H). So
        // two vectors of dpre are live at a time, not the whole segment.
        constexpr int D0 = ((EPV - H) * (int)sizeof(T)) / 4;
        const int prev_lane = (lane + 63) & 63;
        const int next_lane = (lane + 1) & 63;

        // ---- dpre of vector j + dweight/dbias partials ----
        // PART: some lane's vector j may hold a position outside the row
        auto dpre_vec = [&](const int j, float* dpj, auto part_c) {
            constexpr bool PART = decltype(part_c)::value;
            const int32_t t = t0 + (j * 64 + lane) * EPV;
            u32x4 pv = vzero();
#pragma unroll
            for (int d = D0; d < 4; ++d) {
                const uint32_t send = (lane == 63) ? (j > 0 ? v[j > 0 ? j - 1 : 0][d] : 0u) : v[j][d];
                pv[d] = lane_get(send, prev_lane);
            }
            if (j == 0 && lane == 0) pv = h;
            // an aligned row's first vector past its end: its window reads
            // zero too, so that no x of the row meets that vector's zero dpre
            // (zero times a non-finite x would be NaN)
            if (!FULL && !RAG && t >= L) pv = vzero();
            float win[H + EPV];
#pragma unroll
            for (int i = 0; i < H; ++i) {
                if constexpr (FULL || !RAG)  // m == 0 whenever a first segment is full
                    win[i] = (j == 0 && use_init) ? hinit[i] : vget<T>(pv, EPV - H + i);
                else  // before the row: position i - H - m, initial_states slot i - m
                    win[i] = (j == 0 && use_init) ? pick<H>(hinit, i - m) : vget<T>(pv, EPV - H + i);
            }
#pragma unroll
            for (int i = 0; i < EPV; ++i) win[H + i] = vget<T>(v[j], i);
#pragma unroll
            for (int i = 0; i < EPV; ++i) {
                const float g = vget<T>(gv[j], i);
                float d = g;
                if constexpr (SILU) {
                    // q = -log2(e) * pre, from pre-scaled weights and bias
                    float q = bq;
#pragma unroll
                    for (int k = 0; k < W; ++k) q = __builtin_fmaf(wq[k], win[i + k], q);
                    d = silu_bwd_q(g, q);
                }
                // outside the row: dpre is zero and the position adds nothing
                // to the weight gradient (a select, not a product with zero,
                // which a non-finite x there would turn into NaN). Aligned
                // rows end on a vector boundary: the test is the vector's.
                const bool outside = PART && (RAG ? (t + i < m || t + i >= L) : t >= L);
                if (outside) d = 0.0f;
                dpj[i] = d;
                pb += d;
#pragma unroll
                for (int k = 0; k < W; ++k) {
                    const float s = __builtin_fmaf(d, win[i + k], pw[k]);
                    pw[k] = (RAG && outside) ? pw[k] : s;
                }
            }
        };

        // ---- dx of vector j: dpj is its dpre; dpn is vector j + 1's, or for
        //      the last vector dpre of the next segment's first H positions ----
        auto dx_vec = [&](const int j, const float* dpj, const float* dpn) {
            const int32_t t = t0 + (j * 64 + lane) * EPV;
            const bool lastv = j == VPT - 1;
            float de[EPV + H];
#pragma unroll
            for (int i = 0; i < EPV; ++i) de[i] = dpj[i];
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float send = (lane == 0) ? (lastv ? 0.0f : dpn[i]) : dpj[i];
                const float r = lane_get(send, next_lane);
                de[EPV + i] = (lane == 63 && lastv) ? dpn[i] : r;
            }
            float o[EPV];
#pragma unroll
            for (int i = 0; i < EPV; ++i) {
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < W; ++k) acc = __builtin_fmaf(w[W - 1 - k], de[i + k], acc);
                o[i] = acc;
            }
            // dfinal_states tail (_fn.py:308-315): the row's last W-1
            // positions [L - H, L), those inside the row. A wave-uniform
            // branch skips it for every segment without the row end (as a
            // lane-masked block it was issued, empty, by all of them).
            if (dfin_row) {
                if constexpr (!RAG) {  // the row's last vector ends with them
                    const bool last = t + EPV == L;
#pragma unroll
                    for (int i = EPV - H; i < EPV; ++i) {
                        const float v = round_to<T>(o[i]) + dfin[H - EPV + i];
                        o[i] = last ? v : o[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < EPV; ++i) {
                        const int32_t pos = t + i;
                        const float v = round_to<T>(o[i]) + pick<H>(dfin, pos - L + H);
                        o[i] = (pos >= L - H && pos < L && pos >= m) ? v : o[i];
                    }
                }
            }
            if constexpr (!RAG) {
                if (FULL || t < L) vstore_nt(dxr + t, vpack<T>(o));
            } else {
                const u32x4 ov = vpack<T>(o);
                if (FULL || (t >= m && t + EPV <= L)) {
                    vstore_nt(dxr + t, ov);
                } else if (t < L) {  // a vector shared with a neighbouring row
#pragma unroll
                    for (int e = 0; e < EPV; ++e)
                        if ((uint32_t)(t + e - m) < (uint32_t)p.seqlen) st_elem<T>(dxr + t + e, ov, e);
                }
            }
        };

        float dp[2][EPV];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if constexpr (RAG && !FULL && SILU) {
                // With SiLU, x and dout zeroed past the row's end (and before its
                // start, above) make every outside position's dpre an exact zero
                // whenever the row's own values are finite; where they are not,
                // the reference's weight and bias gradients are NaN as well (the
                // SiLU derivative at a non-finite pre is NaN). So no position
                // needs a mask of its own. Wave-uniform test: vector j may hold
                // positions past the end.
                if (t0 + (j + 1) * 64 * EPV > L) {
                    const int32_t t = t0 + (j * 64 + lane) * EPV;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t keep = lead_mask<T>(d, L - t);
                        r.v[j][d] &= keep;
                        r.gv[j][d] &= keep;
                    }
                }
                dpre_vec(j, dp[j & 1], std::false_type{});
            } else if constexpr (RAG && !FULL) {
                // a ragged row's segments are not full, but only their first and
                // last vectors hold positions outside the row (wave-uniform test)
                const int32_t vs = t0 + j * 64 * EPV;  // vector j of lane 0
                if (vs >= m && vs + 64 * EPV <= L) dpre_vec(j, dp[j & 1], std::false_type{});
                else dpre_vec(j, dp[j & 1], std::true_type{});
            } else {
                dpre_vec(j, dp[j & 1], std::bool_constant<!FULL>{});
            }
            if (j == 0 && p.dinitial_states != nullptr && t0 == 0) {  // wave-uniform
                // dinitial_states (bwd_full_cpu/kernel.mojo:210-219) from dpre of
                // positions 0 .. H-1: elements m .. m+H-1 of lane 0's first
                // vector, the ones past its end in lane 1's
                float d0[H];
#pragma unroll
                for (int q = 0; q < H; ++q) {
                    if constexpr (FULL || !RAG) {
                        d0[q] = dp[0][q];
                    } else {
                        const float own = pick<EPV>(dp[0], m + q);
                        const float nxt = __int_as_float(
                            __builtin_amdgcn_readlane(__float_as_int(pick<EPV>(dp[0], m + q - EPV)), 1));
                        d0[q] = m + q < EPV ? own : nxt;
                    }
                }
                if (lane == 0) {
                    T* di = static_cast<T*>(p.dinitial_states) + b * p.dinitial_states_stride[0] +
                            c * p.dinitial_states_stride[1];
#pragma unroll
                    for (int i = 0; i < H; ++i) {
                        float acc = 0.0f;
#pragma unroll
                        for (int k = 0; k <= i; ++k) acc = __builtin_fmaf(w[k], d0[i - k], acc);
                        st(di, i * p.dinitial_states_stride[2], acc);
                    }
                }
            }
            if (j > 0) dx_vec(j - 1, dp[(j - 1) & 1], dp[j & 1]);
        }

        // ---- dpre of the first H positions of the next segment (used by lane 63;
        //      zero when this segment ends the row) ----
        float dn[H];
#pragma unroll
        for (int i = 0; i < H; ++i) dn[i] = 0.0f;
        if (tn < L) {
            float xw[2 * H];
#pragma unroll
            for (int i = 0; i < H; ++i) {
                xw[i] = vget<T>(v[VPT - 1], EPV - H + i);
                xw[H + i] = vget<T>(xn, i);
            }
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float g = vget<T>(gn, i);
                float d = g;
                if constexpr (SILU) {
                    float q = bq;
#pragma unroll
                    for (int k = 0; k < W; ++k) q = __builtin_fmaf(wq[k], xw[i + k], q);
                    d = silu_bwd_q(g, q);
                }
                if (tn + i >= L) d = 0.0f;
                dn[i] = d;
            }
        }
        dx_vec(VPT - 1, dp[(VPT - 1) & 1], dn);
    }
}

// The seq_idx form of bwd_rows_compute (seq_idx excludes initial_states,
// dfinal_states and dinitial_states, so none of those appear). dx is
// scattered instead of gathered: the gates of position s -- tap k is kept
// when seq_idx[s - k] == seq_idx[s] -- are compared once, while s's dpre is
// computed, and used at once for the SiLU argument, the weight-gradient
// sums and s's contributions w[W-1-k] * dpre[s] to dx[s - k]. No gate is
// kept beyond its position (a gather compares each pair a second time, for
// dx, and keeps the comparisons or the ids of both sides until then).
// Contributions to the H positions before the lane's first collect in a
// carry that the owning lane fetches from its neighbour (lane 63: from lane
// 0 of the next vector, or from the next segment's first H positions); each
// dx sum is the gather's fma chain with that carry added as one term.
template <typename T, int W, int VPT, bool SILU, bool FULL, bool RAG>
__device__ __forceinline__ void bwd_rows_compute_seq(const cc1d_bwd_params& p, int lane, int64_t b, int64_t c,
                                                     int32_t t0, int32_t m, RowTile<VPT> r,
                                                     const float* w, const float* wq, float bq, float* pw,
                                                     float& pb) {
    constexpr int EPV = elems16<T>::value;
    constexpr int H = W - 1;
    constexpr int SEG = 64 * VPT * EPV;
    static_assert(H <= EPV, "the halo must fit in one 16-byte vector");
    constexpr int D0 = ((EPV - H) * (int)sizeof(T)) / 4;
    const int32_t Lr = (int32_t)p.seqlen;  // the row's length
    const int32_t L = Lr + m;              // its end: the row is [m, L) in these positions
    const int32_t tn = t0 + SEG;  // first position of the next segment
    T* __restrict__ dxr = static_cast<T*>(p.dx) + b * p.dx_stride[0] + c * p.dx_stride[1] - m;
    const int32_t* __restrict__ sr = p.seq_idx + b * p.seq_idx_stride[0];
    // (unit time stride) ragged rows: a vector's ids start rid ids past a
    // 16-byte boundary (its first position, t - m, is a multiple of 4 plus
    // -m); the row's first id a0 past one
    const int a0 = RAG ? (int)uniform32((uint32_t)(reinterpret_cast<uintptr_t>(sr) / 4) & 3u) : 0;
    const int rid = (a0 - m) & 3;
    const int prev_lane = (lane + 63) & 63;
    const int next_lane = (lane + 1) & 63;
    // a ragged row's first vector holds m elements of the previous row: x
    // there reads as zero, as before an aligned row (a padding position's id
    // matches theirs, -1, and a tap is kept by its id alone)
    if (RAG && !FULL && t0 == 0 && m > 0 && lane == 0) {
        float fx[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e) fx[e] = e >= m ? vget<T>(r.v[0], e) : 0.0f;
        r.v[0] = vpack<T>(fx);
    }

    // ids: the lane's positions (-1 outside the row), and the H before and
    // after the segment (wave-uniform, -1 outside the row)
    int32_t id[VPT][EPV];
    IdsRaw<EPV> raw[RAG ? VPT : 1];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        if constexpr (!RAG) {  // 16-byte vectors of 4 ids
#pragma unroll
            for (int q = 0; q < EPV / 4; ++q) {
                const u32x4 sv = (FULL || t < L) ? *reinterpret_cast<const u32x4*>(sr + t + 4 * q)
                                                 : u32x4{0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
#pragma unroll
                for (int e = 0; e < 4; ++e) id[j][4 * q + e] = (int32_t)sv[e];
            }
        } else {
            ids_load<EPV, !FULL>(sr, Lr, t - m, rid, a0, raw[j]);
        }
    }
    if constexpr (RAG) {  // -1 outside the row
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int32_t pos = t0 + (j * 64 + lane) * EPV - m;
            const int32_t vs = t0 + j * 64 * EPV;  // vector j of lane 0: inside the row in every lane?
            if (FULL || (vs >= m && vs + 64 * EPV <= L)) ids_shift<EPV, false>(raw[j], Lr, pos, rid, id[j]);
            else ids_shift<EPV, true>(raw[j], Lr, pos, rid, id[j]);
        }
    }
    int32_t hid[H], nid[H];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        const int32_t ph = t0 - H + i - m, pn = tn + i - m;  // row positions
        hid[i] = ph >= 0 ? ld_uniform(sr + ph) : -1;
        nid[i] = pn < Lr ? ld_uniform(sr + pn) : -1;
    }

    float acc[2][EPV];  // dx sums of the lane's positions, by vector parity
    float carry[2][H];  // contributions to the H positions before the lane's first

    // dx of vector j: add the carries for its last H positions (from the next
    // lane's vector j; lane 63: `nxt`, lane 0's carry of vector j + 1, or with
    // `local` the next segment's contributions computed by every lane) and store
    auto finish = [&](const int j, float* a, const float* cj, const float* nxt, const bool local) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float send = (lane == 0 && !local) ? nxt[i] : cj[i];
            float rv = lane_get(send, next_lane);
            if (local && lane == 63) rv = nxt[i];
            a[EPV - H + i] += rv;
        }
        if constexpr (!RAG) {
            if (FULL || t < L) vstore_nt(dxr + t, vpack<T>(a));
        } else if (FULL || (t >= m && t + EPV <= L)) {
            vstore_nt(dxr + t, vpack<T>(a));
        } else if (t < L) {  // a vector shared with a neighbouring row
#pragma unroll
            for (int e = 0; e < EPV; ++e)
                if (t + e >= m && t + e < L) st(dxr, t + e, a[e]);
        }
    };

#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int32_t t = t0 + (j * 64 + lane) * EPV;
        // x and id windows: the H positions before the vector, then its EPV
        u32x4 pv = vzero();
#pragma unroll
        for (int d = D0; d < 4; ++d) {
            const uint32_t send = (lane == 63) ? (j > 0 ? r.v[j > 0 ? j - 1 : 0][d] : 0u) : r.v[j][d];
            pv[d] = lane_get(send, prev_lane);
        }
        if (j == 0 && lane == 0) pv = r.h;
        float win[H + EPV];
        int32_t iw[H + EPV];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            win[i] = vget<T>(pv, EPV - H + i);
            const int32_t send = (lane == 63) ? (j > 0 ? id[j > 0 ? j - 1 : 0][EPV - H + i] : -1)
                                              : id[j][EPV - H + i];
            const int32_t rv = lane_get(send, prev_lane);
            iw[i] = (j == 0 && lane == 0) ? hid[i] : rv;
        }
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
            win[H + i] = vget<T>(r.v[j], i);
            iw[H + i] = id[j][i];
        }
        float* a = acc[j & 1];
        float* cr = carry[j & 1];
#pragma unroll
        for (int i = 0; i < EPV; ++i) a[i] = 0.0f;
#pragma unroll
        for (int i = 0; i < H; ++i) cr[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            const int32_t cur = iw[H + e];
            // tap kk of position s covers s - (H - kk): kept when the ids match
            bool keep[W];
            float xe[W];
#pragma unroll
            for (int kk = 0; kk < H; ++kk) {
                keep[kk] = iw[e + kk] == cur;
                xe[kk] = keep[kk] ? win[e + kk] : 0.0f;
            }
            keep[H] = true;
            xe[H] = win[H + e];
            const float g = vget<T>(r.gv[j], e);
            float d = g;
            if constexpr (SILU) {
                float q = bq;
#pragma unroll
                for (int kk = 0; kk < W; ++kk) q = __builtin_fmaf(wq[kk], xe[kk], q);
                d = silu_bwd_q(g, q);
            }
            // outside the row: nothing added (a select, as in bwd_rows_compute)
            const bool outside = !FULL && (RAG ? (t + e < m || t + e >= L) : t + e >= L);
            if (outside || cur < 0) d = 0.0f;
            pb += d;
#pragma unroll
            for (int kk = 0; kk < W; ++kk) {
                const float s = __builtin_fmaf(d, xe[kk], pw[kk]);
                pw[kk] = outside ? pw[kk] : s;
            }
            // dx[s - k] += w[W-1-k] * dpre[s] where tap W-1-k of s is kept
#pragma unroll
            for (int k = 0; k <= H; ++k) {
                const float de = keep[H - k] ? d : 0.0f;
                if (e - k >= 0) a[e - k] = __builtin_fmaf(w[W - 1 - k], de, a[e - k]);
                else cr[H + e - k] = __builtin_fmaf(w[W - 1 - k], de, cr[H + e - k]);
            }
            // one position at a time: the sums are updated here (the compiler
            // would otherwise sink their fmas to the end, keeping every
            // position's gated window alive until then)
#pragma unroll
            for (int kk = 0; kk < W; ++kk) asm volatile("" : "+v"(pw[kk]));
            asm volatile("" : "+v"(pb));
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j > 0) finish(j - 1, acc[(j - 1) & 1], carry[(j - 1) & 1], carry[j & 1], false);
    }

    // contributions of the next segment's first H positions to this segment's
    // last H (lane 63's; zero when this segment ends the row)
    float cn[H];
#pragma unroll
    for (int i = 0; i < H; ++i) cn[i] = 0.0f;
    if (tn < L) {
        float xw[2 * H];
        int32_t iw[2 * H];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            xw[i] = vget<T>(r.v[VPT - 1], EPV - H + i);
            xw[H + i] = vget<T>(r.xn, i);
            iw[i] = id[VPT - 1][EPV - H + i];
            iw[H + i] = nid[i];
        }
#pragma unroll
        for (int s2 = 0; s2 < H; ++s2) {
            const int32_t cur = iw[H + s2];
            const float g = vget<T>(r.gn, s2);
            float d = g;
            if constexpr (SILU) {
                float q = bq;
#pragma unroll
                for (int kk = 0; kk < W; ++kk) {
                    const bool keep = kk == H || iw[s2 + kk] == cur;
                    q = __builtin_fmaf(wq[kk], keep ? xw[s2 + kk] : 0.0f, q);
                }
                d = silu_bwd_q(g, q);
            }
            if (tn + s2 >= L || cur < 0) d = 0.0f;
            // to the positions before tn: k = s2 + 1 .. H, position index H + s2 - k
#pragma unroll
            for (int k = s2 + 1; k <= H; ++k) {
                const float de = iw[H + s2 - k] == cur ? d : 0.0f;
                cn[H + s2 - k] = __builtin_fmaf(w[W - 1 - k], de, cn[H + s2 - k]);
            }
        }
    }
    finish(VPT - 1, acc[(VPT - 1) & 1], carry[(VPT - 1) & 1], cn, true);
}

// One (row, segment) item: the tile's loads go out first, then the halo,
// weight and bias reads (scalar loads, issued together: the bias address is
// always valid, so no branch holds them apart), which all complete before
// the arithmetic starts -- the empty asm uses their values, so the compiler
// can neither sink a load into the arithmetic nor wait for each on its own.
template <typename T, int W, int VPT, bool SILU, bool SEQ, bool FULL, bool RAG>
__device__ __forceinline__ void bwd_rows_item(const cc1d_bwd_params& p, int lane, int64_t b, int64_t c, int32_t t0,
                                              int32_t m, float* pw, float& pb) {
    RowTile<VPT> r;
    bwd_rows_load<T, VPT, FULL>(p, lane, b, c, t0, m, r);
    float w[W];
    const T* __restrict__ wr = static_cast<const T*>(p.weight) + c * p.weight_stride[0];
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = ld_uniform(wr + k * p.weight_stride[1]);
    const T* br = p.bias ? static_cast<const T*>(p.bias) + c * p.bias_stride : static_cast<const T*>(p.weight);
    const float braw = ld_uniform(br);
#pragma unroll
    for (int k = 0; k < W; ++k) asm volatile("" ::"s"(w[k]));
    asm volatile("" ::"s"(braw), "s"(r.h), "s"(r.xn), "s"(r.gn));
    __builtin_amdgcn_sched_barrier(0);
    const float bias = p.bias ? braw : 0.0f;
    // the pre-scaled weights are wave-uniform: kept in scalar registers
    float wq[W];
#pragma unroll
    for (int k = 0; k < W; ++k) wq[k] = uniform_f32(-kLog2e * w[k]);
    const float bq = uniform_f32(-kLog2e * bias);
    if constexpr (SEQ) bwd_rows_compute_seq<T, W, VPT, SILU, FULL, RAG>(p, lane, b, c, t0, m, r, w, wq, bq, pw, pb);
    else bwd_rows_compute<T, W, VPT, SILU, FULL, RAG>(p, lane, b, c, t0, m, r, w, wq, bq, pw, pb);
}

// One (row, segment) item per wavefront, kRowsWPB per block; item = (row,
// segment) with row = b * dim + c, in memory order like the forward, so
// consecutive wavefronts stream consecutive rows. The wavefront sums its
// weight/bias-gradient partials with DPP adds, and lanes 0..W add them to
// the fp32 accumulators (one atomic instruction) or write the item's partial
// record. All index arithmetic is 32-bit (the launcher checks the ranges).
// (A channel order -- one block per channel, its batch entries' sums added
// in LDS and written in the dtype, so the typed backward needs no second
// launch -- measured 2 us slower at C2: the block's rows lie in B regions
// of the tensors instead of one.)
template <typename T, int W, int VPT, bool SILU, bool SEQ, bool RAG>
__global__ void __launch_bounds__(64 * kRowsWPB) bwd_rows_vec(const BwdArgs a) {
    constexpr int SEG = 64 * VPT * elems16<T>::value;
    const cc1d_bwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const uint32_t item = uniform32(blockIdx.x * (uint32_t)kRowsWPB + (threadIdx.x >> 6));
    if (item >= (uint32_t)a.n_items) return;
    // (row, segment) and (b, c) by the host's invariant-divisor constants:
    // scalar multiply-shifts, no division on the vector unit
    const uint32_t row = a.nseg_div.div(item);
    const int32_t t0 = (int32_t)((item - row * (uint32_t)a.nseg) * SEG);
    const uint32_t b = a.dim_div.div(row);
    const uint32_t c = row - b * (uint32_t)p.dim;
    float pw[W];
#pragma unroll
    for (int k = 0; k < W; ++k) pw[k] = 0.0f;
    float pb = 0.0f;
    constexpr int EPV = elems16<T>::value;
    // ragged rows: the row starts m elements past a 16-byte boundary
    int32_t m = 0;
    if constexpr (RAG) {
        const T* xrow = static_cast<const T*>(p.x) + (int64_t)b * p.x_stride[0] + (int64_t)c * p.x_stride[1];
        m = (int32_t)uniform32((uint32_t)(reinterpret_cast<uintptr_t>(xrow) / sizeof(T)) & (EPV - 1));
    }
    const int32_t Lv = (int32_t)p.seqlen + m;
    // a ragged row's last segment may lie past its end: it adds nothing but
    // still writes its (zero) record
    if ((t0 > 0 || m == 0) && t0 + SEG <= Lv)
        bwd_rows_item<T, W, VPT, SILU, SEQ, true, RAG>(p, lane, b, c, t0, m, pw, pb);
    else if (!RAG || t0 < Lv)
        bwd_rows_item<T, W, VPT, SILU, SEQ, false, RAG>(p, lane, b, c, t0, m, pw, pb);

    // ---- weight / bias gradient: wavefront sum, then lanes 0..W add ----
    float mine = wave_sum(pb);
#pragma unroll
    for (int k = 0; k < W; ++k) {
        const float s = wave_sum(pw[k]);
        if (lane == k) mine = s;
    }
    if (a.part != nullptr) {  // record (W taps, bias) of this item
        if (lane <= W) a.part[(int64_t)item * (W + 1) + lane] = mine;
    } else if (lane < W) {
        unsafeAtomicAdd(p.dweight_acc + (int64_t)c * p.dweight_acc_stride[0] + lane * p.dweight_acc_stride[1], mine);
    } else if (lane == W && p.dbias_acc != nullptr) {
        unsafeAtomicAdd(p.dbias_acc + (int64_t)c * p.dbias_acc_stride, mine);
    }
}

// One channel c of batch b over steps [t0, t1), any strides: writes dx (and
// dinitial_states when t0 == 0) and returns the chunk's weight/bias-gradient
// partials in pw / pb. Windows of the previous W-1 positions are rolled in
// registers; the step loop is not unrolled, so the register footprint is
// small.
template <typename T, int W, bool SILU>
__device__ __forceinline__ void bwd_chunk(const cc1d_bwd_params& p, int64_t b, int64_t c, int64_t t0, int64_t t1,
                                          float* pw, float& pb) {
    constexpr int H = W - 1;
    const int64_t L = p.seqlen;
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    const T* __restrict__ gr = static_cast<const T*>(p.dout) + b * p.dout_stride[0] + c * p.dout_stride[1];
    T* __restrict__ dxr = static_cast<T*>(p.dx) + b * p.dx_stride[0] + c * p.dx_stride[1];
    const int32_t* sr = p.seq_idx ? p.seq_idx + b * p.seq_idx_stride[0] : nullptr;
    const T* ir = p.initial_states ? static_cast<const T*>(p.initial_states) + b * p.initial_states_stride[0] +
                                         c * p.initial_states_stride[1]
                                   : nullptr;

    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        w[k] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;

    // Windows over positions s-H..s: x values, seq ids, dpre values.
    float xw[W], dw[W];
    int32_t iw[W];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        const int64_t s = t0 - H + i;
        if (s >= 0) xw[i] = ld(xr, s * p.x_stride[2]);
        else xw[i] = ir ? ld(ir, (s + H) * p.initial_states_stride[2]) : 0.0f;
        iw[i] = (sr != nullptr && s >= 0) ? sr[s * p.seq_idx_stride[1]] : -1;
        dw[i] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < W; ++k) pw[k] = 0.0f;
    pb = 0.0f;
    float dfirst[H];
#pragma unroll
    for (int i = 0; i < H; ++i) dfirst[i] = 0.0f;

    const int64_t m = (H < L) ? H : L;  // dfinal tail length
    for (int64_t s = t0; s < t1 + H; ++s) {
        const bool in = s < L;
        xw[H] = in ? ld(xr, s * p.x_stride[2]) : 0.0f;
        iw[H] = (in && sr != nullptr) ? sr[s * p.seq_idx_stride[1]] : -1;
        float d = 0.0f;
        if (in) {
            const float g = ld(gr, s * p.dout_stride[2]);
            d = g;
            if (SILU) {
                float pre = bias;
#pragma unroll
                for (int k = 0; k < W; ++k)
                    if (sr == nullptr || iw[k] == iw[H]) pre = __builtin_fmaf(w[k], xw[k], pre);
                d = g * silu_grad(pre);
            }
            if (sr != nullptr && iw[H] < 0) d = 0.0f;
        }
        dw[H] = d;
        if (s < t1) {
            pb += d;
#pragma unroll
            for (int k = 0; k < W; ++k)  // a tap before the row adds a term only with initial_states
                if ((sr == nullptr || iw[k] == iw[H]) && (ir != nullptr || s + k >= H))
                    pw[k] = __builtin_fmaf(d, xw[k], pw[k]);
#pragma unroll
            for (int i = 0; i < H; ++i)
                if (s == i) dfirst[i] = d;
        }
        const int64_t q = s - H;
        if (q >= t0) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < W; ++k)
                if (sr == nullptr || iw[k] == iw[0]) acc = __builtin_fmaf(w[W - 1 - k], dw[k], acc);
            if (p.dfinal_states != nullptr && q >= L - m)
                acc = round_to<T>(acc) + ld(static_cast<const T*>(p.dfinal_states),
                                            b * p.dfinal_states_stride[0] + c * p.dfinal_states_stride[1] +
                                                (q - L + H) * p.dfinal_states_stride[2]);
            st(dxr, q * p.dx_stride[2], acc);
        }
#pragma unroll
        for (int i = 0; i < H; ++i) {
            xw[i] = xw[i + 1];
            iw[i] = iw[i + 1];
            dw[i] = dw[i + 1];
        }
    }
    if (p.dinitial_states != nullptr && t0 == 0) {
        T* di = static_cast<T*>(p.dinitial_states) + b * p.dinitial_states_stride[0] + c * p.dinitial_states_stride[1];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k <= i; ++k) acc = __builtin_fmaf(w[k], dfirst[i - k], acc);
            st(di, i * p.dinitial_states_stride[2], acc);
        }
    }
}

// ---- channel-last (unit channel stride) backward: a walk along time ------
//
// A lane owns CPL adjacent channels (4 bytes) and a wavefront the 64 * CPL
// channels of one run of R time steps [t0, t0 + R). The wavefront walks its
// run in chunks of G steps, one 256-byte row of x and of dout per load
// instruction, the next chunk's loads in flight while the current chunk is
// computed. x and dpre of the last H = W - 1 positions slide in registers;
// dx of position s is emitted once dpre[s + H] is known, so a run computes
// dpre for [t0, t0 + R + H) (a tail of H steps, the next run's first) and
// emits dx for [t0, t0 + R). Loads are unconditional at positions clamped
// into [0, L); a chunk whose window lies inside the sequence with one
// seq_idx id (>= 0) takes the ungated arithmetic, any other chunk the same
// steps with every condition applied (all of them wave-uniform: one time
// step per instruction row, the ids in scalar registers). Index arithmetic
// is 32-bit inside a batch (the launcher checks the ranges).
//
// Launch shape (C3, 8192 x 4096 bf16): chunks of 4 steps, runs of 128, 8
// runs per block -- 2048 wavefronts, two per SIMD: 39.1-39.7 / 37.9-38.2 us
// (seq_idx / initial_states); the same access pattern with no arithmetic
// takes 34.1-34.4 us. Measured against it in the same sessions: runs of 64
// steps (8 or 16 per block) 46.0 / 42.0 us and of 96 54.9 us for seq_idx;
// three chunks in flight instead of one 43.1 / 42.0; the block order
// remapped to XCDs 41.4-41.7 for seq_idx; four wavefronts sharing each
// chunk's 1 KB row pieces through LDS (16 bytes per lane, a barrier per
// chunk) 41.7 / 40.3 at best; and, with no arithmetic, 8-byte lanes no
// faster than these 4-byte ones (34.4 us). The earlier tile kernel (16
// steps loaded at once, 4 per block) took 46.3 / 45.0.

// The weights and bias of a lane's channels, kept raw: they are read before
// the walk and converted where they are used, so no conversion waits for
// them (memory counters retire in order) ahead of the first chunk's loads.
// Without a bias the bias read goes to x's first element (an unconditional
// load, so no branch waits on it) and bias() returns zero.
template <typename T, int W, int CPL> struct ClWeights {
    T w[W][CPL], b[CPL];
    bool has_bias;
    __device__ __forceinline__ void load(const cc1d_bwd_params& p, int32_t c0, bool active) {
        const T* __restrict__ wp = static_cast<const T*>(p.weight);
        has_bias = p.bias != nullptr;
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
            const int64_t c = active ? c0 + e : 0;
#pragma unroll
            for (int k = 0; k < W; ++k) w[k][e] = wp[c * p.weight_stride[0] + k * p.weight_stride[1]];
            const T* bsrc = has_bias ? static_cast<const T*>(p.bias) + c * p.bias_stride : static_cast<const T*>(p.x);
            b[e] = *bsrc;
        }
    }
    __device__ __forceinline__ float bias(int e) const { return has_bias ? to_f32(b[e]) : 0.0f; }
};

// G rows of x and dout from position c0 on, raw; ids[i]: seq_idx at position
// c0 - H + i (clamped into [0, L)), read through the scalar cache (NI = G + H
// with seq_idx, else 1 unused).
template <typename T, int CPL, int G, int NI> struct ClChunk {
    Lanes<T, CPL> x[G], g[G];
    int32_t ids[NI];
};

// Sliding state of a walk: x and dpre at the H positions before the current
// one (x zero before the sequence or initial_states there, dpre zero before
// the run), and the weight/bias-gradient partial sums.
template <int W, int CPL> struct ClWalk {
    float xw[W - 1][CPL], dw[W - 1][CPL];
    float pw[W][CPL], pb[CPL];
    // Ends a step's partial-sum updates where they are written: otherwise the
    // compiler sinks each running sum's fma towards its next use (the next
    // step's), until a chunk's updates all sit at its end and every step's
    // dpre and x stay live until then.
    __device__ __forceinline__ void pin_sums() {
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
#pragma unroll
            for (int k = 0; k < W; ++k) asm volatile("" : "+v"(pw[k][e]));
            asm volatile("" : "+v"(pb[e]));
        }
    }
};

// One dword of a row at byte offset off from the wavefront-uniform base
// (offsets below 2^32: the launcher checks the ranges). A 64-bit uniform base
// plus a 32-bit per-lane offset is the scalar-base form of the global
// access (global_load_dword v, v_off, s[base]): one 32-bit add per access.
// Non-temporal: a walk reads each row once (the few rows a neighbouring run
// reads again are its H-row prime and tail); at C3 the backward took 37.3 /
// 38.5 us with non-temporal row loads against 40.5 / 41.3 us with cached ones.
template <typename T, int CPL> __device__ __forceinline__ Lanes<T, CPL> row_load(const T* base, uint32_t off) {
    static_assert(Lanes<T, CPL>::ND == 1, "one dword per lane");
    Lanes<T, CPL> v;
    v.d[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(base) + off));
    return v;
}
template <typename T, int CPL> __device__ __forceinline__ void row_store_nt(T* base, uint32_t off, const Lanes<T, CPL>& v) {
    static_assert(Lanes<T, CPL>::ND == 1, "one dword per lane");
    __builtin_nontemporal_store(v.d[0], reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(base) + off));
}

// Kernel: the WPB wavefronts of a block take WPB consecutive runs of the same
// channels; their weight/bias-gradient partials are summed through LDS and
// the block adds the sums with fp32 atomics on consecutive addresses (or
// writes them as its record). Block order: channel group fastest, then run
// group, then batch.
template <typename T, int W, int G, int R, int WPB, bool SILU, bool SEQ>
__global__ void __launch_bounds__(64 * WPB) bwd_clw(const BwdArgs a) {
    constexpr int CPL = 4 / (int)sizeof(T);
    constexpr int H = W - 1;
    constexpr int NC = 64 * CPL;  // channels per wavefront
    constexpr int NCH = R / G;    // chunks per run
    static_assert(R == G || (R % (2 * G) == 0 && R >= 2 * G), "one chunk, or chunks in pairs");
    static_assert(G >= H, "the first chunk covers the H steps whose dx belongs to the previous run");
    using Chunk = ClChunk<T, CPL, G, SEQ ? G + H : 1>;
    __shared__ float red[WPB][NC * (W + 1)];
    const cc1d_bwd_params& p = a.p;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // (the divisions run on the vector unit; uniform32 brings the results
    // back to scalar registers, so every pointer derived from them is scalar)
    const uint32_t ngroups = (uint32_t)a.groups, ntgroups = (uint32_t)a.nseg;
    const uint32_t grp = uniform32(blockIdx.x % ngroups);
    const uint32_t rest = uniform32(blockIdx.x / ngroups);
    const uint32_t tg = uniform32(rest % ntgroups);
    const uint32_t b = uniform32(rest / ntgroups);
    const int32_t L = (int32_t)p.seqlen;
    const int32_t t0 = (int32_t)uniform32((tg * WPB + wave) * R);
    const int32_t cw0 = (int32_t)(grp * NC);
    const int32_t c0 = cw0 + lane * CPL;
    const bool active = c0 < (int32_t)p.dim;

    ClWalk<W, CPL> s;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
        s.pb[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) s.pw[k][e] = 0.0f;
    }
    if (t0 < L) {  // runs past the end only join the block reduction
        const int32_t xs2 = (int32_t)p.x_stride[2], gs2 = (int32_t)p.dout_stride[2];
        const int32_t ds2 = (int32_t)p.dx_stride[2];
        // lanes past the last channel read channel 0 of the group's rows (in
        // bounds); they store nothing and their partials are dropped
        const int32_t lo = active ? lane * CPL : 0;
        const uint32_t lob = (uint32_t)lo * (uint32_t)sizeof(T);  // the lane's byte offset in a row
        const T* __restrict__ xb = static_cast<const T*>(p.x) + b * p.x_stride[0] + cw0;
        const T* __restrict__ gb = static_cast<const T*>(p.dout) + b * p.dout_stride[0] + cw0;
        T* __restrict__ dxb = static_cast<T*>(p.dx) + b * p.dx_stride[0] + cw0;
        const int32_t* __restrict__ sr = SEQ ? p.seq_idx + b * p.seq_idx_stride[0] : nullptr;
        const int32_t ss1 = SEQ ? (int32_t)p.seq_idx_stride[1] : 0;
        auto clampL = [&](int32_t t) { return t < 0 ? 0 : (t < L ? t : L - 1); };

        // loads of the rows of chunk c (NR of them) and of its id window
        auto load = [&](int32_t cs, Chunk& ch, auto nr) {
            constexpr int NR = decltype(nr)::value;
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                const int32_t t = clampL(cs + j);
                ch.x[j] = row_load<T, CPL>(xb, (uint32_t)(t * xs2) * (uint32_t)sizeof(T) + lob);
                ch.g[j] = row_load<T, CPL>(gb, (uint32_t)(t * gs2) * (uint32_t)sizeof(T) + lob);
            }
            if constexpr (SEQ) {
                constexpr int NI = G + H;
                if (ss1 == 1 && cs >= H && cs - H + NI <= L) {
                    // the window's ids are consecutive and in range: one scalar load
                    const __attribute__((address_space(4))) int32_t* q =
                        (const __attribute__((address_space(4))) int32_t*)reinterpret_cast<uintptr_t>(sr + (cs - H));
#pragma unroll
                    for (int i = 0; i < NI; ++i) ch.ids[i] = q[i];
                } else {
#pragma unroll
                    for (int i = 0; i < NI; ++i) ch.ids[i] = ld_uniform(sr + clampL(cs - H + i) * ss1);
                }
            }
        };

        // x rows t0-H .. t0-1 (zero before the sequence, or initial_states)
        Lanes<T, CPL> prime[H];
        const bool prime_rows = t0 >= H;
        if (prime_rows) {
#pragma unroll
            for (int k = 0; k < H; ++k)
                prime[k] = row_load<T, CPL>(xb, (uint32_t)((t0 - H + k) * xs2) * (uint32_t)sizeof(T) + lob);
        }
        ClWeights<T, W, CPL> wt;
        wt.load(p, c0, active);
        Chunk A, B;
        load(t0, A, std::integral_constant<int, G>{});

        // w for dx; wq, bq (scaled by -log2(e)) give the SiLU argument q = -log2(e) * pre
        // directly, as the exponent silu_bwd_q takes
        float w[W][CPL], wq[W][CPL], bq[CPL];
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
#pragma unroll
            for (int k = 0; k < W; ++k) {
                w[k][e] = to_f32(wt.w[k][e]);
                wq[k][e] = -kLog2e * w[k][e];
            }
            bq[e] = -kLog2e * wt.bias(e);
        }
#pragma unroll
        for (int k = 0; k < H; ++k) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                s.xw[k][e] = prime_rows ? prime[k].get(e) : 0.0f;
                s.dw[k][e] = 0.0f;
            }
        }
        if (!prime_rows && p.initial_states != nullptr && active) {  // t0 == 0
            const int32_t cl = opaque(c0);
#pragma unroll
            for (int k = 0; k < H; ++k)
#pragma unroll
                for (int e = 0; e < CPL; ++e)
                    s.xw[k][e] = ld(static_cast<const T*>(p.initial_states),
                                    b * p.initial_states_stride[0] + (cl + e) * p.initial_states_stride[1] +
                                        k * p.initial_states_stride[2]);
        }
        const int32_t m = H < L ? H : L;  // dfinal tail length

        // shift the windows by one position: x and dpre of the current step enter
        auto slide = [&](const float* xc, const float* dn) {
#pragma unroll
            for (int k = 0; k + 1 < H; ++k)
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    s.xw[k][e] = s.xw[k + 1][e];
                    s.dw[k][e] = s.dw[k + 1][e];
                }
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                s.xw[H - 1][e] = xc[e];
                s.dw[H - 1][e] = dn[e];
            }
        };
        auto store_dx = [&](int32_t pos, const float* o) {
            Lanes<T, CPL> ov;
            ov.set(o);
            row_store_nt<T, CPL>(dxb, (uint32_t)(pos * ds2) * (uint32_t)sizeof(T) + lob, ov);
        };

        // NS steps of chunk ch at cs, ungated (the chunk's window [cs-H, cs+NS+H)
        // lies in [0, L) with one id); ACC: the steps are the run's own;
        // HEAD: the run's first chunk (dx before the run belongs to the
        // previous one)
        auto steps_clean = [&](const Chunk& ch, int32_t cs, auto ns, auto accc, auto headc) {
            constexpr int NS = decltype(ns)::value;
            constexpr bool ACC = decltype(accc)::value;
            constexpr bool HEAD = decltype(headc)::value;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                float xc[CPL], dn[CPL], o[CPL];
                const Lanes<T, CPL> xl = ch.x[j], gl = ch.g[j];
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    xc[e] = xl.get(e);
                    const float gval = gl.get(e);
                    float d = gval;
                    if constexpr (SILU) {
                        float q = bq[e];
#pragma unroll
                        for (int k = 0; k < H; ++k) q = __builtin_fmaf(wq[k][e], s.xw[k][e], q);
                        q = __builtin_fmaf(wq[H][e], xc[e], q);
                        d = silu_bwd_q(gval, q);
                    }
                    dn[e] = d;
                    if constexpr (ACC) {
                        s.pb[e] += d;
#pragma unroll
                        for (int k = 0; k < H; ++k) s.pw[k][e] = __builtin_fmaf(d, s.xw[k][e], s.pw[k][e]);
                        s.pw[H][e] = __builtin_fmaf(d, xc[e], s.pw[H][e]);
                    }
                    // dx at position cs + j - H: dpre there .. here, taps w[H] .. w[0]
                    float acc = 0.0f;
#pragma unroll
                    for (int k = 0; k < H; ++k) acc = __builtin_fmaf(w[H - k][e], s.dw[k][e], acc);
                    o[e] = __builtin_fmaf(w[0][e], d, acc);
                }
                if (active && (j >= H || !HEAD)) store_dx(cs + j - H, o);
                slide(xc, dn);
                if constexpr (ACC) s.pin_sums();
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // the same steps with every condition: positions past the end,
        // seq_idx gates, dfinal_states, dinitial_states (chunk 0 of run 0)
        auto steps_gated = [&](const Chunk& ch, int32_t cs, auto ns, auto accc) {
            constexpr int NS = decltype(ns)::value;
            constexpr bool ACC = decltype(accc)::value;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const int32_t pos = cs + j;
                const bool in = pos < L;
                int32_t idk[H], idp = 0;  // ids of the window positions and of pos
                if constexpr (SEQ) {
#pragma unroll
                    for (int k = 0; k < H; ++k) idk[k] = ch.ids[j + k];
                    idp = ch.ids[j + H];
                } else {
#pragma unroll
                    for (int k = 0; k < H; ++k) idk[k] = 0;
                }
                const bool dead = !in || idp < 0;
                float xc[CPL], dn[CPL];
                const Lanes<T, CPL> xl = ch.x[j], gl = ch.g[j];
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    xc[e] = in ? xl.get(e) : 0.0f;
                    const float gval = gl.get(e);
                    float d = gval;
                    if constexpr (SILU) {
                        float q = bq[e];
#pragma unroll
                        for (int k = 0; k < H; ++k)
                            if (idk[k] == idp) q = __builtin_fmaf(wq[k][e], s.xw[k][e], q);
                        q = __builtin_fmaf(wq[H][e], xc[e], q);
                        d = silu_bwd_q(gval, q);
                    }
                    if (dead) d = 0.0f;
                    dn[e] = d;
                    // a step past the end adds no term (zero dpre times a
                    // non-finite x of the window would be NaN), nor does a tap
                    // before the row without initial_states; padding inside
                    // the sequence adds its zero terms, as the reference does
                    // (wave-uniform tests)
                    if (ACC && in) {
                        s.pb[e] += d;
#pragma unroll
                        for (int k = 0; k < H; ++k)
                            if (idk[k] == idp && (pos + k >= H || p.initial_states != nullptr))
                                s.pw[k][e] = __builtin_fmaf(d, s.xw[k][e], s.pw[k][e]);
                        s.pw[H][e] = __builtin_fmaf(d, xc[e], s.pw[H][e]);
                    }
                }
                // dx at position sp = pos - H: tap k kept when id(sp + k) == id(sp)
                const int32_t sp = pos - H;
                if (sp >= t0 && sp < L && active) {
                    float o[CPL];
#pragma unroll
                    for (int e = 0; e < CPL; ++e) {
                        float acc = 0.0f;
#pragma unroll
                        for (int k = 0; k < H; ++k)
                            if (idk[k] == idk[0]) acc = __builtin_fmaf(w[H - k][e], s.dw[k][e], acc);
                        if (idp == idk[0]) acc = __builtin_fmaf(w[0][e], dn[e], acc);
                        o[e] = acc;
                    }
                    if (p.dfinal_states != nullptr && sp >= L - m) {
                        const int32_t cl = opaque(c0);
#pragma unroll
                        for (int e = 0; e < CPL; ++e)
                            o[e] = round_to<T>(o[e]) + ld(static_cast<const T*>(p.dfinal_states),
                                                          b * p.dfinal_states_stride[0] +
                                                              (cl + e) * p.dfinal_states_stride[1] +
                                                              (sp - L + H) * p.dfinal_states_stride[2]);
                    }
                    store_dx(sp, o);
                }
                slide(xc, dn);
                if constexpr (ACC) s.pin_sums();
                // dinitial_states (bwd_full_cpu/kernel.mojo:210-219): once the
                // window holds dpre[0 .. H-1] (position H-1 is step H-1 of the
                // chunk at 0, as chunks start at multiples of G >= H)
                if (j == H - 1 && cs == 0 && p.dinitial_states != nullptr && active) {
                    const int32_t cl = opaque(c0);
#pragma unroll
                    for (int e = 0; e < CPL; ++e) {
                        T* di = static_cast<T*>(p.dinitial_states) + b * p.dinitial_states_stride[0] +
                                (cl + e) * p.dinitial_states_stride[1];
#pragma unroll
                        for (int i = 0; i < H; ++i) {
                            float acc = 0.0f;
#pragma unroll
                            for (int k = 0; k <= i; ++k) acc = __builtin_fmaf(w[k][e], s.dw[i - k][e], acc);
                            st(di, i * p.dinitial_states_stride[2], acc);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // a chunk is clean when its window [cs-H, cs+NS+H) lies inside the
        // sequence (the last H positions: dfinal_states reach back that far)
        // and, with seq_idx, carries one id >= 0
        auto steps = [&](const Chunk& ch, int32_t cs, auto ns, auto accc, auto headc) {
            constexpr int NS = decltype(ns)::value;
            bool clean = cs >= H && cs + NS + H <= L;
            if constexpr (SEQ) {
                const int32_t id0 = ch.ids[0];
                bool same = id0 >= 0;
#pragma unroll
                for (int i = 1; i < NS + H; ++i) same = same && ch.ids[i] == id0;
                clean = clean && same;
            }
            if (clean) steps_clean(ch, cs, ns, accc, headc);
            else steps_gated(ch, cs, ns, accc);
        };

        constexpr std::integral_constant<int, G> kG{};
        constexpr std::integral_constant<int, H> kH{};
        constexpr std::true_type kAcc{};
        constexpr std::false_type kNoAcc{};
        constexpr std::true_type kHead{};
        constexpr std::false_type kBody{};
        if constexpr (NCH == 1) {
            // the whole run at once: its rows and the tail's are all in flight
            load(t0 + R, B, kH);  // the tail: the next run's first H rows
            steps(A, t0, kG, kAcc, kHead);
            steps(B, t0 + R, kH, kNoAcc, kBody);
        } else {
            // chunk 0 in A, chunk 1 in B; then chunks in pairs, each buffer
            // refilled as soon as it has been consumed; the tail last
            load(t0 + G, B, kG);
            steps(A, t0, kG, kAcc, kHead);
#pragma unroll 1
            for (int c = 1; c + 1 < NCH; c += 2) {
                const int32_t cb = t0 + c * G;
                load(cb + G, A, kG);
                steps(B, cb, kG, kAcc, kBody);
                load(cb + 2 * G, B, kG);
                steps(A, cb + G, kG, kAcc, kBody);
            }
            load(t0 + R, A, kH);  // the tail: the next run's first H rows
            steps(B, t0 + R - G, kG, kAcc, kBody);
            steps(A, t0 + R, kH, kNoAcc, kBody);
        }
        if (!active) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                s.pb[e] = 0.0f;
#pragma unroll
                for (int k = 0; k < W; ++k) s.pw[k][e] = 0.0f;
            }
        }
    }

    // ---- weight / bias gradient: sum the block's runs in LDS, then
    //      consecutive fp32 atomics (or the block's record) ----
    float* rr = red[wave];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
#pragma unroll
        for (int k = 0; k < W; ++k) rr[(lane * CPL + e) * W + k] = s.pw[k][e];
        rr[NC * W + lane * CPL + e] = s.pb[e];
    }
    __syncthreads();
    constexpr int NE = NC * (W + 1);
    for (int idx = threadIdx.x; idx < NE; idx += 64 * WPB) {
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < WPB; ++q) sum += red[q][idx];
        if (a.part != nullptr) {  // the block's record: NC channels x W taps, then NC bias sums
            a.part[(int64_t)blockIdx.x * NE + idx] = sum;
        } else if (idx < NC * W) {
            const int32_t c = cw0 + idx / W;
            if (c < (int32_t)p.dim)
                unsafeAtomicAdd(p.dweight_acc + c * p.dweight_acc_stride[0] + (idx % W) * p.dweight_acc_stride[1], sum);
        } else if (p.dbias_acc != nullptr) {
            const int32_t c = cw0 + (idx - NC * W);
            if (c < (int32_t)p.dim) unsafeAtomicAdd(p.dbias_acc + c * p.dbias_acc_stride, sum);
        }
    }
}

template <typename T, int W, bool SILU>
__global__ void __launch_bounds__(256) bwd_generic(const BwdArgs a) {
    constexpr int H = W - 1;
    const cc1d_bwd_params& p = a.p;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n_items) return;
    const int64_t c = idx % p.dim;
    const int64_t rest = idx / p.dim;
    const int64_t ch = rest % a.nseg;
    const int64_t b = rest / a.nseg;
    const int64_t t0 = ch * a.chunk;
    const int64_t t1 = (t0 + a.chunk < p.seqlen) ? t0 + a.chunk : p.seqlen;
    float pw[W], pb;
    bwd_chunk<T, W, SILU>(p, b, c, t0, t1, pw, pb);
    (void)H;
    if (a.part != nullptr) {  // record (W taps, bias) of this thread's chunk
#pragma unroll
        for (int k = 0; k < W; ++k) a.part[idx * (W + 1) + k] = pw[k];
        a.part[idx * (W + 1) + W] = pb;
        return;
    }
#pragma unroll
    for (int k = 0; k < W; ++k)
        unsafeAtomicAdd(p.dweight_acc + c * p.dweight_acc_stride[0] + k * p.dweight_acc_stride[1], pw[k]);
    if (p.dbias_acc != nullptr) unsafeAtomicAdd(p.dbias_acc + c * p.dbias_acc_stride, pb);
}

namespace {

template <typename T>
bool rows_vec_ok(const cc1d_bwd_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    if (p.width - 1 > EPV) return false;
    if (p.x_stride[2] != 1 || p.dout_stride[2] != 1 || p.dx_stride[2] != 1) return false;
    if (p.seqlen % EPV != 0) return false;
    if (!aligned16(p.x) || !aligned16(p.dout) || !aligned16(p.dx)) return false;
    if (p.x_stride[0] % EPV || p.x_stride[1] % EPV || p.dout_stride[0] % EPV || p.dout_stride[1] % EPV ||
        p.dx_stride[0] % EPV || p.dx_stride[1] % EPV)
        return false;
    if (p.seq_idx != nullptr &&
        (p.seq_idx_stride[1] != 1 || p.seq_idx_stride[0] % 4 != 0 || !aligned16(p.seq_idx)))
        return false;
    // 32-bit index arithmetic: positions and items (one block each) must fit
    if (p.seqlen + 64 * 4 * EPV >= ((int64_t)1 << 31)) return false;
    if (p.batch * p.dim * ceil_div(p.seqlen, 64 * EPV) >= ((int64_t)1 << 31)) return false;
    return true;
}

// ragged rows (a seqlen that is not a multiple of the vector, or rows that do
// not start on a 16-byte boundary): unit time stride, and dout and dx laid out
// like x modulo the vector -- the same element strides modulo EPV and bases a
// multiple of 16 bytes apart -- so every row of each starts as far past a
// 16-byte boundary as its row of x; seq_idx with a unit time stride
template <typename T>
bool rows_ragged_ok(const cc1d_bwd_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    if (p.width - 1 > EPV) return false;
    if (p.x_stride[2] != 1 || p.dout_stride[2] != 1 || p.dx_stride[2] != 1) return false;
    for (const int64_t* s : {p.dout_stride, p.dx_stride})
        if ((s[0] - p.x_stride[0]) % EPV != 0 || (s[1] - p.x_stride[1]) % EPV != 0) return false;
    const intptr_t x = reinterpret_cast<intptr_t>(p.x);
    if ((reinterpret_cast<intptr_t>(p.dout) - x) % 16 != 0 || (reinterpret_cast<intptr_t>(p.dx) - x) % 16 != 0)
        return false;
    if (p.seq_idx != nullptr && (p.seq_idx_stride[1] != 1 || reinterpret_cast<uintptr_t>(p.seq_idx) % 4 != 0))
        return false;
    const int64_t lim = (int64_t)1 << 31;
    if (p.seqlen + 64 * 4 * EPV + EPV >= lim) return false;
    if (p.batch * p.dim * ceil_div(p.seqlen + EPV, 64 * EPV) >= lim) return false;
    return true;
}

// channel-last tiles: unit channel stride, CPL | dim, rows aligned to the
// CPL-channel lane vector, 32-bit positions inside a batch
template <typename T, int CPL>
bool cl_ok(const cc1d_bwd_params& p) {
    constexpr int64_t NB = CPL * (int64_t)sizeof(T);
    if (p.x_stride[1] != 1 || p.dout_stride[1] != 1 || p.dx_stride[1] != 1) return false;
    if (p.dim % CPL != 0) return false;
    if ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.dout) |
         reinterpret_cast<uintptr_t>(p.dx)) % NB)
        return false;
    if (p.x_stride[0] % CPL || p.x_stride[2] % CPL || p.dout_stride[0] % CPL || p.dout_stride[2] % CPL ||
        p.dx_stride[0] % CPL || p.dx_stride[2] % CPL)
        return false;
    const int64_t span = p.seqlen + kClWPB * kClR + 16;  // past the furthest run start
    const int64_t lim = (int64_t)1 << 31;
    if (p.dim >= lim || span * p.x_stride[2] >= lim || span * p.dout_stride[2] >= lim || span * p.dx_stride[2] >= lim)
        return false;
    // row offsets are formed in bytes as 32-bit unsigned values (position *
    // stride * sizeof(T) + the lane's bytes): an fp32 batch entry of 2^30 or
    // more elements takes the 64-bit generic kernel
    const int64_t blim = ((int64_t)1 << 32) - 64 * NB;
    if (span * p.x_stride[2] * (int64_t)sizeof(T) >= blim || span * p.dout_stride[2] * (int64_t)sizeof(T) >= blim ||
        span * p.dx_stride[2] * (int64_t)sizeof(T) >= blim)
        return false;
    if (p.seq_idx != nullptr && span * p.seq_idx_stride[1] >= lim) return false;
    if (p.batch * ceil_div(p.dim / CPL, 64) * ceil_div(p.seqlen, kClR * kClWPB) >= lim) return false;
    return true;
}


// ---- launch planning ----------------------------------------------------

enum BwdKind { kBwdRows = 0, kBwdCl = 1, kBwdGeneric = 2 };

// Kernel choice and launch geometry for one call; shared by the launch, the
// workspace size and the partial-sum reduction.
struct BwdPlan {
    int kind;
    int vpt;           // rows: 16-byte vectors per lane
    int cpl;           // cl: channels per lane
    BwdArgs a;
    int64_t blocks;
    int64_t records;   // partial-sum records (rows / generic: items; cl: blocks)
    int64_t rec_floats;
};

template <typename T, int W>
BwdPlan plan_bwd(const cc1d_bwd_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    BwdPlan pl;
    pl.a.p = p;
    pl.a.part = nullptr;
    pl.a.chunk = 0;
    pl.a.groups = 0;
    pl.vpt = 0;
    pl.cpl = 0;
    pl.rec_floats = W + 1;
    pl.a.ragged = 0;
    const bool aligned = W - 1 <= EPV && rows_vec_ok<T>(p);
    if (aligned || (W - 1 <= EPV && rows_ragged_ok<T>(p))) {
        pl.a.ragged = aligned ? 0 : 1;
        // vectors a row spans: a ragged row may start up to EPV - 1 elements
        // past a vector boundary
        const int64_t nvec = aligned ? p.seqlen / EPV : ceil_div(p.seqlen + EPV - 1, EPV);
        const int64_t per = ceil_div(nvec, 64);
        pl.kind = kBwdRows;
        // vectors per lane (measured at C2's batch and dim): 4 from 129 vectors
        // a row on -- one segment of 4 beats two of 2, the same lane slots
        // (L = 1536: 38.8 instead of 45.2 us), when the grid keeps 2048
        // wavefronts (on smaller grids the more wavefronts of 2 measured faster)
        // -- except when a row a little longer
        // than a multiple of the 4-vector segment would leave its last one
        // mostly empty: 2 when that takes at most 85 % of the lane slots
        // (L = 2056: 58.8 instead of 65.7 us; 4104: 99.8 instead of 105.2)
        const int64_t rows = p.batch * p.dim;
        pl.vpt = per >= 4 || (per == 3 && rows >= 2048) ? 4 : (per >= 2 ? 2 : 1);
        if (pl.vpt == 4 && ceil_div(nvec, 128) * 128 * 100 <= ceil_div(nvec, 256) * 256 * 85) pl.vpt = 2;
        pl.a.nseg = ceil_div(nvec, 64 * (int64_t)pl.vpt);
        pl.a.n_items = p.batch * p.dim * pl.a.nseg;
        pl.a.nseg_div = FastDiv((uint32_t)pl.a.nseg);
        pl.a.dim_div = FastDiv((uint32_t)p.dim);
        pl.blocks = ceil_div(pl.a.n_items, (int64_t)kRowsWPB);
        pl.records = pl.a.n_items;
        return pl;
    }
    constexpr int CPL = 4 / (int)sizeof(T);
    if (cl_ok<T, CPL>(p)) {
        pl.kind = kBwdCl;
        pl.cpl = CPL;
        pl.a.groups = ceil_div(p.dim / CPL, 64);
        // run length: a wavefront walks its run chunk by chunk, each chunk's
        // loads in flight behind the previous one's arithmetic, so a run takes
        // about the same time at any problem size (memory latency per chunk);
        // the longest run that still gives 2048 wavefronts (2 per SIMD), else
        // the shortest (measured, bf16, B = 1: D = 4096, L = 8192 keeps 128;
        // D = 4096, L = 4096: 24.9 us with 64 against 35.2 with 128; D = 1536,
        // L = 2048: 9.1 us with 16 against 34.9 with 128)
        pl.a.chunk = kClRShort;
        for (const int r : {kClR, kClRMid}) {
            if (p.batch * pl.a.groups * ceil_div(p.seqlen, (int64_t)r) >= 2048) {
                pl.a.chunk = r;
                break;
            }
        }
        pl.a.nseg = ceil_div(p.seqlen, pl.a.chunk * kClWPB);  // run groups per row
        pl.a.n_items = 0;
        pl.blocks = p.batch * pl.a.groups * pl.a.nseg;
        pl.records = pl.blocks;
        pl.rec_floats = 64 * CPL * (W + 1);
        return pl;
    }
    pl.kind = kBwdGeneric;
    pl.a.chunk = 64;
    pl.a.nseg = ceil_div(p.seqlen, pl.a.chunk);
    pl.a.n_items = p.batch * p.dim * pl.a.nseg;
    pl.blocks = ceil_div(pl.a.n_items, 256);
    pl.records = pl.a.n_items;
    return pl;
}

template <typename T, int W, bool SILU>
int launch_plan(const BwdPlan& pl, const cc1d_bwd_params& p, hipStream_t stream) {
    const dim3 grid((unsigned)pl.blocks);
    const BwdArgs& a = pl.a;
    if (pl.kind == kBwdRows) {
        if constexpr (W - 1 <= elems16<T>::value) {
            return with_flag(p.seq_idx != nullptr, [&](auto qc) {
                constexpr bool SEQ = decltype(qc)::value;
                const dim3 block(64 * kRowsWPB);
                return with_flag(a.ragged != 0, [&](auto rc) {
                    constexpr bool RAG = decltype(rc)::value;
                    if (pl.vpt == 4) return launch(bwd_rows_vec<T, W, 4, SILU, SEQ, RAG>, grid, block, stream, a);
                    if (pl.vpt == 2) return launch(bwd_rows_vec<T, W, 2, SILU, SEQ, RAG>, grid, block, stream, a);
                    return launch(bwd_rows_vec<T, W, 1, SILU, SEQ, RAG>, grid, block, stream, a);
                });
            });
        }
        return CC1D_ERR_SHAPE;  // not reached: the plan only picks rows when the halo fits
    }
    if (pl.kind == kBwdCl) {
        return with_flag(p.seq_idx != nullptr, [&](auto qc) {
            constexpr bool SEQ = decltype(qc)::value;
            constexpr int G = W - 1 <= kClG ? kClG : 2 * kClG;  // at least H steps per chunk
            const dim3 block(64 * kClWPB);
            if (a.chunk == kClRShort) return launch(bwd_clw<T, W, G, kClRShort, kClWPB, SILU, SEQ>, grid, block, stream, a);
            if (a.chunk == kClRMid) return launch(bwd_clw<T, W, G, kClRMid, kClWPB, SILU, SEQ>, grid, block, stream, a);
            return launch(bwd_clw<T, W, G, kClR, kClWPB, SILU, SEQ>, grid, block, stream, a);
        });
    }
    return launch(bwd_generic<T, W, SILU>, grid, dim3(256), stream, a);
}

// Sum of the partial records of each channel, in a fixed order, written in
// the dtype. Lanes run along the values of a record, so every load of a
// wavefront reads 64 consecutive floats: value o of the outputs is (channel
// o / (W+1), tap o % (W+1), the bias as tap W) for row and generic records,
// whose (W+1) values per channel are contiguous, and value f of a channel
// group's record (NC x W taps, then NC biases) for channel-last records.
// Wavefront q of a block takes records q, q + waves, ... in that order, RB of
// them in flight at a time, and the block adds its wavefronts' sums in LDS in
// wavefront order. (With a lane per channel reading values 16-20 bytes
// apart, C3's records took 8-10 us.)
struct RedArgs {
    const float* part;
    void* dweight;
    void* dbias;
    int64_t dweight_stride[2];
    int64_t dbias_stride;
    int64_t batch, dim, nseg, groups;
    int nc;           // cl: channels per record
    int64_t nout;     // values reduced: dim * (W+1) (rows, generic) or groups * nc * (W+1) (cl)
};

template <typename T, int W, int KIND>
__global__ void __launch_bounds__(1024) bwd_reduce(const RedArgs r) {
    constexpr int RB = 8;  // records in flight per wavefront
    __shared__ float acc[16][64];
    const int lane = threadIdx.x & 63;
    const int q = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int64_t o = (int64_t)blockIdx.x * 64 + lane;  // output value of this lane
    const int64_t n = r.batch * r.nseg;                  // records per channel
    const bool on = o < r.nout;
    // channel, tap (W: bias) and the offset of this value in record j = (b, g)
    int64_t c, k, grp = 0, f = 0;
    if constexpr (KIND == kBwdCl) {
        const int64_t rec = (int64_t)r.nc * (W + 1);
        grp = o / rec;
        f = o - grp * rec;
        const bool tap = f < (int64_t)r.nc * W;
        c = grp * r.nc + (tap ? f / W : f - (int64_t)r.nc * W);
        k = tap ? f % W : W;
    } else {
        c = o / (W + 1);
        k = o - c * (W + 1);
    }
    auto at = [&](int64_t j) -> const float* {
        const int64_t b = j / r.nseg, g = j - b * r.nseg;
        if constexpr (KIND == kBwdCl)
            return r.part + ((b * r.nseg + g) * r.groups + grp) * (int64_t)r.nc * (W + 1) + f;
        else if constexpr (KIND == kBwdRows)
            return r.part + ((b * r.dim + c) * r.nseg + g) * (W + 1) + k;
        else
            return r.part + ((b * r.nseg + g) * r.dim + c) * (W + 1) + k;
    };
    float sum = 0.0f;
    if (on) {
        for (int64_t jb = q; jb < n; jb += (int64_t)nw * RB) {
            float v[RB];
#pragma unroll
            for (int u = 0; u < RB; ++u) {
                const int64_t j = jb + (int64_t)u * nw;
                v[u] = j < n ? *at(j) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < RB; ++u) sum += v[u];
        }
    }
    acc[q][lane] = sum;
    __syncthreads();
    if (q == 0 && on && c < r.dim) {
        float t = 0.0f;
        for (int w = 0; w < nw; ++w) t += acc[w][lane];
        if (k < W) st(static_cast<T*>(r.dweight), c * r.dweight_stride[0] + k * r.dweight_stride[1], t);
        else if (r.dbias != nullptr) st(static_cast<T*>(r.dbias), c * r.dbias_stride, t);
    }
}

// The same sums when a channel has at most kRedSmall records (C2: 4): one
// wavefront per 64 output values, each lane loads all of its value's records
// at once and adds them in record order -- the order bwd_reduce uses, so
// both give the same bits -- with no LDS step and no barrier.
constexpr int kRedSmall = 16;

template <typename T, int W, int KIND>
__global__ void __launch_bounds__(64) bwd_reduce_small(const RedArgs r) {
    const int64_t o = (int64_t)blockIdx.x * 64 + threadIdx.x;  // output value of this lane
    if (o >= r.nout) return;
    const int64_t n = r.batch * r.nseg;  // records per channel (<= kRedSmall)
    int64_t c, k, grp = 0, f = 0;
    if constexpr (KIND == kBwdCl) {
        const int64_t rec = (int64_t)r.nc * (W + 1);
        grp = o / rec;
        f = o - grp * rec;
        const bool tap = f < (int64_t)r.nc * W;
        c = grp * r.nc + (tap ? f / W : f - (int64_t)r.nc * W);
        k = tap ? f % W : W;
    } else {
        c = o / (W + 1);
        k = o - c * (W + 1);
    }
    float v[kRedSmall];
#pragma unroll
    for (int j = 0; j < kRedSmall; ++j) {
        v[j] = 0.0f;
        if (j < n) {
            const int64_t b = j / r.nseg, g = j - b * r.nseg;
            const float* q;
            if constexpr (KIND == kBwdCl)
                q = r.part + ((b * r.nseg + g) * r.groups + grp) * (int64_t)r.nc * (W + 1) + f;
            else if constexpr (KIND == kBwdRows)
                q = r.part + ((b * r.dim + c) * r.nseg + g) * (W + 1) + k;
            else
                q = r.part + ((b * r.nseg + g) * r.dim + c) * (W + 1) + k;
            v[j] = *q;
        }
    }
    if (c >= r.dim) return;
    float t = 0.0f;
#pragma unroll
    for (int j = 0; j < kRedSmall; ++j)
        if (j < n) t += v[j];
    if (k < W) st(static_cast<T*>(r.dweight), c * r.dweight_stride[0] + k * r.dweight_stride[1], t);
    else if (r.dbias != nullptr) st(static_cast<T*>(r.dbias), c * r.dbias_stride, t);
}

}  // namespace

// ---- per-dtype entry templates (instantiated by cc1d_bwd_<dtype>.hip) ----

template <typename T>
int launch_bwd_dtype(const cc1d_bwd_params& p, hipStream_t stream) {
    return with_width(p.width, [&](auto wc) {
        constexpr int W = decltype(wc)::value;
        return with_flag(p.apply_silu != 0, [&](auto sc) {
            const BwdPlan pl = plan_bwd<T, W>(p);
            return launch_plan<T, W, decltype(sc)::value>(pl, p, stream);
        });
    });
}

template <typename T>
int64_t bwd_workspace_floats_dtype(const cc1d_bwd_params& p) {
    int64_t n = -1;
    with_width(p.width, [&](auto wc) {
        const BwdPlan pl = plan_bwd<T, decltype(wc)::value>(p);
        n = pl.records * pl.rec_floats;
        return (int)CC1D_OK;
    });
    return n;
}

template <typename T>
int launch_bwd_typed_dtype(const cc1d_bwd_params& p, const cc1d_bwd_grads& g, hipStream_t stream) {
    return with_width(p.width, [&](auto wc) {
        constexpr int W = decltype(wc)::value;
        return with_flag(p.apply_silu != 0, [&](auto sc) {
            BwdPlan pl = plan_bwd<T, W>(p);
            if (pl.records * pl.rec_floats > g.workspace_floats) return (int)CC1D_ERR_WORKSPACE;
            if (g.workspace == nullptr) return (int)CC1D_ERR_NULL_POINTER;
            pl.a.part = g.workspace;
            const int st = launch_plan<T, W, decltype(sc)::value>(pl, p, stream);
            if (st != CC1D_OK) return st;
            RedArgs r;
            r.part = g.workspace;
            r.dweight = g.dweight;
            r.dbias = g.dbias;
            r.dweight_stride[0] = g.dweight_stride[0];
            r.dweight_stride[1] = g.dweight_stride[1];
            r.dbias_stride = g.dbias_stride;
            r.batch = p.batch;
            r.dim = p.dim;
            r.nseg = pl.a.nseg;
            r.groups = pl.a.groups;
            r.nc = 64 * (pl.cpl > 0 ? pl.cpl : 1);
            r.nout = pl.kind == kBwdCl ? pl.a.groups * r.nc * (W + 1) : p.dim * (W + 1);
            const int64_t n = p.batch * pl.a.nseg;  // records per channel
            const dim3 grid((unsigned)ceil_div(r.nout, 64));
            if (n <= kRedSmall) {
                const dim3 one(64);
                if (pl.kind == kBwdRows) return launch(bwd_reduce_small<T, W, kBwdRows>, grid, one, stream, r);
                if (pl.kind == kBwdCl) return launch(bwd_reduce_small<T, W, kBwdCl>, grid, one, stream, r);
                return launch(bwd_reduce_small<T, W, kBwdGeneric>, grid, one, stream, r);
            }
            const dim3 threads(64 * (unsigned)(n < 16 ? n : 16));
            if (pl.kind == kBwdRows) return launch(bwd_reduce<T, W, kBwdRows>, grid, threads, stream, r);
            if (pl.kind == kBwdCl) return launch(bwd_reduce<T, W, kBwdCl>, grid, threads, stream, r);
            return launch(bwd_reduce<T, W, kBwdGeneric>, grid, threads, stream, r);
        });
    });
}

}  // namespace cc1d
