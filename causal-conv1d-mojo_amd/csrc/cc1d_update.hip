// cc1d_update.hip -- decode (single-token / short-burst) update kernels.
//
// Semantics (src/causal_conv1d_mojo/update_cpu/kernel.mojo:49-141):
//   full = cat(history, x[b,c,0:seqlen]) where history is the W-1 values
//   before the write head: state[-(W-1):] (linear) or
//   state[(cs - (W-1) + j) mod S] with cs = cache_seqlens[b] mod S (circular).
//   out[i] = act(bias + sum_k w[k] * full[i+k])
//   linear:   state <- last S values of cat(state, x)
//   circular: state[(cs + i) mod S] <- x[i]
//   conv_state_indices redirect the state row; a negative (padding) or
//   out-of-pool index zeroes out[b] and leaves the pool untouched.
//
// Kernels
//   update_dir     -- linear mode, one token, S == W-1 <= 4, channel-contiguous
//                     x / out and contiguous state rows: a lane owns one dword
//                     of x (2 bf16/fp16 channels, 1 fp32) of two batch
//                     entries and loads the channels' state span (H dwords)
//                     directly, one load per span; no LDS; four wavefronts
//                     (channel groups) per workgroup.
//   update_lin     -- the same for W > 5: one token, S == W-1, channel-contiguous x /
//                     out and contiguous state rows: one wavefront per (batch
//                     entry, 16 * EPV channels) moves the group's state and x
//                     spans as consecutive 16-byte vectors, one per lane at
//                     W = 4, and exchanges them through LDS.
//   update_circ_vec -- circular mode on contiguous state lines of whole
//                     16-byte chunks: two adjacent lanes per (b, c) read the
//                     two chunks that hold its window (one 32-byte access),
//                     swap them, and write back the ones the window touches.
//   update_circ    -- other circular cases with up to 8 new tokens; one thread
//                     per (b, c) with all loads issued before any store.
//   update_generic -- everything else; one thread per (b, c).
// Both use the forward's tap loop (fma in k order, then SiLU), so a decode
// loop reproduces the full forward bit for bit.
#include "cc1d_internal.hpp"

namespace cc1d {

struct UpdArgs {
    cc1d_update_params p;
    int64_t n_items;
};

__device__ __forceinline__ int64_t state_row(const cc1d_update_params& p, int64_t b) {
    if (p.conv_state_indices == nullptr) return b;
    const int64_t r = p.conv_state_indices[b];
    return (r < 0 || r >= p.state_rows) ? -1 : r;
}

template <typename T, int W, bool SILU, bool CIRC>
__global__ void __launch_bounds__(256) update_generic(const UpdArgs a) {
    constexpr int H = W - 1;
    const cc1d_update_params& p = a.p;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n_items) return;
    const int64_t c = idx % p.dim;
    const int64_t b = idx / p.dim;
    const int64_t Ls = p.seqlen;
    const int64_t S = p.state_len;
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];
    const int64_t row = state_row(p, b);
    if (row < 0) {
        for (int64_t i = 0; i < Ls; ++i) st(orow, i * p.out_stride[2], 0.0f);
        return;
    }
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    T* __restrict__ sr = static_cast<T*>(p.conv_state) + row * p.conv_state_stride[0] + c * p.conv_state_stride[1];
    const int64_t ss = p.conv_state_stride[2];
    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        w[k] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;

    float win[W];
    int64_t head = 0;
    if constexpr (CIRC) {
        int64_t cs = (int64_t)p.cache_seqlens[b] % S;
        if (cs < 0) cs += S;  // floored modulo (torch.remainder)
        head = cs - H;
        if (head < 0) head += S;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            win[i] = ld(sr, head * ss);
            if (++head >= S) head -= S;
        }
    } else {
        // shift left by Ls, keeping the W-1 history values in registers
        for (int64_t i = 0; i < S - Ls - H; ++i) sr[i * ss] = sr[(i + Ls) * ss];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const T v = sr[(S - H + i) * ss];
            const int64_t wi = S - Ls - H + i;
            if (wi >= 0) sr[wi * ss] = v;
            win[i] = to_f32(v);
        }
    }
    for (int64_t i = 0; i < Ls; ++i) {
        const T xv = xr[i * p.x_stride[2]];
        if constexpr (CIRC) {
            sr[head * ss] = xv;
            if (++head >= S) head -= S;
        } else {
            const int64_t wi = S - Ls + i;
            if (wi >= 0) sr[wi * ss] = xv;
        }
        win[H] = to_f32(xv);
        float acc = conv_taps<W>(bias, w, win);
        if constexpr (SILU) acc = silu(acc);
        st(orow, i * p.out_stride[2], acc);
#pragma unroll
        for (int k = 0; k < H; ++k) win[k] = win[k + 1];
    }
}

// Arguments of update_lin: only what it reads, packed so that one batch of
// scalar loads fetches all of them (the full params struct took two
// dependent rounds of kernel-argument loads before the first data load).
template <typename T> struct LinArgs {
    const T* x;
    const T* weight;
    const T* bias;
    T* conv_state;
    const int32_t* idx;
    T* out;
    uint32_t x_row, out_row, state_row;  // row strides (elements) of x, out, the state pool
    uint32_t dim;
    int32_t state_rows;
    uint32_t nbatch;  // batch entries (update_dir)
};

// Linear mode, seqlen 1, state_len == W-1 (H), channel-contiguous x / out and
// contiguous state rows. One wavefront per (batch entry, group of
// NCH = 16 * EPV * NV channels): the group's state span (NCH * H elements) and
// its x span (NCH elements) are 16 * W * NV vectors of 16 bytes, [state | x],
// and lane l loads vectors l, l + 64, ... of that segment, so every load and store
// instruction of the wavefront covers consecutive 16-byte vectors (a lane
// owning whole channels instead reads H vectors at a stride of H vectors:
// ~1 us slower at C4a). x, the weights and the bias are loaded first, then
// the pool index (a scalar load) that the state loads wait for. The segment goes
// through LDS so that each lane takes the H * NV dwords of state and the NV
// dwords of x of its channels (2 NV for 16-bit types, NV for fp32), computes
// their outputs and new state, and puts them back; the stores read the segment back
// in vector order. The state shift moves raw bits, so state values are kept
// bit for bit. The grid is (channel groups, batch entries).
template <typename T, int W, int NV, bool SILU, bool HAS_BIAS, bool HAS_IDX>
__global__ void __launch_bounds__(64) update_lin(const LinArgs<T> a) {
    constexpr int EPV = elems16<T>::value;
    constexpr int H = W - 1;
    constexpr int NCH = 16 * EPV * NV;       // channels per wavefront
    constexpr int NSV = 16 * H * NV;         // state vectors in the segment
    constexpr int NTV = 16 * W * NV;         // all vectors (state, then x)
    constexpr int NSLOT = (NTV + 63) / 64;   // vectors per lane
    constexpr int CPL = EPV / 4 * NV;        // channels per lane
    constexpr int XD = NV;                   // dwords of x (and of out) per lane
    constexpr int SD = H * NV;               // dwords of state per lane
    __shared__ u32x4 seg[64 * NSLOT];
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.y;            // batch entry
    const uint32_t c0 = blockIdx.x * NCH;     // first channel of the group
    const uint32_t nch = min(a.dim - c0, (uint32_t)NCH);  // channels of this group
    const int32_t nxv = (int32_t)(nch / EPV), nsv = (int32_t)(nch * H / EPV);  // valid x / state vectors
    const T* xr = a.x + (size_t)b * a.x_row + c0;
    // Every lane of a slot that holds x vectors loads one, unconditionally: a
    // lane of the state part (or past the group's end) reads an in-bounds x
    // vector of the group and drops it. With no branch around them, the
    // loads are issued before the pool index arrives.
    u32x4 xv[NSLOT];
#pragma unroll
    for (int j = 0; j < NSLOT; ++j) {
        if (64 * j + 63 >= NSV) {  // compile-time after unrolling
            const int32_t xi = min(max((int32_t)(64 * j + lane) - NSV, 0), nxv - 1);
            xv[j] = vload(xr + xi * EPV);
        }
    }
    // this lane's channels: weights (CPL * W elements, XD * W dwords) and bias (XD dwords)
    const uint32_t cl = c0 + CPL * lane;
    const uint32_t cw = cl < a.dim ? cl : 0;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(a.weight + (size_t)cw * W);
    uint32_t wd[XD * W];
#pragma unroll
    for (int k = 0; k < XD * W; ++k) wd[k] = wp[k];
    uint32_t bd[XD];
#pragma unroll
    for (int k = 0; k < XD; ++k) bd[k] = HAS_BIAS ? reinterpret_cast<const uint32_t*>(a.bias + cw)[k] : 0u;
    // the pool index (a scalar load) after the index-free loads, which are
    // then all in flight while the state addresses wait for it; the
    // scheduling fence keeps the compiler from hoisting the index load and
    // its wait above them
    __builtin_amdgcn_sched_barrier(0);
    int32_t row = (int32_t)b;
    if constexpr (HAS_IDX) {
        row = ld_uniform(a.idx + b);
        if (row < 0 || row >= a.state_rows) row = -1;  // padding (any negative) or out of the pool
    }
    // state vectors, also unconditional (a padding entry reads row 0, lanes
    // past the state part an in-bounds vector; both are dropped)
    T* sp = a.conv_state + (size_t)(row >= 0 ? row : 0) * a.state_row + (size_t)c0 * H;
#pragma unroll
    for (int j = 0; j < NSLOT; ++j) {
        const int32_t vi = 64 * j + lane;
        u32x4 v = vzero();
        if (64 * j < NSV) v = vload(sp + min(vi, nsv - 1) * EPV);
        if (64 * j + 63 >= NSV) v = vi >= NSV ? xv[j] : v;
        seg[64 * j + lane] = v;
    }
    __builtin_amdgcn_wave_barrier();
    uint32_t* sd = reinterpret_cast<uint32_t*>(seg);
    uint32_t st[SD], xd[XD];
#pragma unroll
    for (int i = 0; i < SD; ++i) st[i] = sd[SD * lane + i];
#pragma unroll
    for (int i = 0; i < XD; ++i) xd[i] = sd[4 * NSV + XD * lane + i];
    // element n of a dword array: half (n & 1) of dword n / 2 (16-bit) or dword n (fp32)
    auto elem = [&](const uint32_t* d, int n) -> uint32_t {
        if constexpr (EPV == 4) return d[n];
        else return (n & 1) ? (d[n >> 1] >> 16) : (d[n >> 1] & 0xffffu);
    };
    auto as_f32 = [&](uint32_t bits) -> float {
        if constexpr (EPV == 4) return __uint_as_float(bits);
        else return to_f32(T{(uint16_t)bits});
    };
    uint32_t nd[SD], od[XD];
    {
        uint32_t sraw[CPL * H], nraw[CPL * H];
#pragma unroll
        for (int n = 0; n < CPL * H; ++n) sraw[n] = elem(st, n);
        float o[CPL];
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
            const uint32_t xb = elem(xd, e);
            float win[W], w[W];
#pragma unroll
            for (int i = 0; i < H; ++i) win[i] = as_f32(sraw[e * H + i]);
            win[H] = as_f32(xb);
#pragma unroll
            for (int k = 0; k < W; ++k) w[k] = as_f32(elem(wd, e * W + k));
            const float bias = HAS_BIAS ? as_f32(elem(bd, e)) : 0.0f;
            float acc = conv_taps<W>(bias, w, win);
            if constexpr (SILU) acc = silu(acc);
            o[e] = acc;
#pragma unroll
            for (int i = 0; i < H; ++i) nraw[e * H + i] = i + 1 < H ? sraw[e * H + i + 1] : xb;
        }
        if constexpr (EPV == 4) {
#pragma unroll
            for (int i = 0; i < SD; ++i) nd[i] = nraw[i];
#pragma unroll
            for (int i = 0; i < XD; ++i) od[i] = __float_as_uint(o[i]);
        } else {
#pragma unroll
            for (int i = 0; i < SD; ++i) nd[i] = nraw[2 * i] | (nraw[2 * i + 1] << 16);
#pragma unroll
            for (int i = 0; i < XD; ++i) od[i] = pack2<T>(o[2 * i], o[2 * i + 1]);
        }
        if (row < 0) {  // padding entry: zero output, state untouched
#pragma unroll
            for (int i = 0; i < XD; ++i) od[i] = 0u;
        }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < SD; ++i) sd[SD * lane + i] = nd[i];
#pragma unroll
    for (int i = 0; i < XD; ++i) sd[4 * NSV + XD * lane + i] = od[i];
    __builtin_amdgcn_wave_barrier();
    T* orow = a.out + (size_t)b * a.out_row + c0;
#pragma unroll
    for (int j = 0; j < NSLOT; ++j) {
        const int32_t vi = 64 * j + lane;
        if (vi >= NTV) continue;
        const u32x4 r = seg[vi];
        if (vi < NSV) {
            if (row >= 0 && vi < nsv) vstore(sp + vi * EPV, r);
        } else if (vi - NSV < nxv) {
            vstore(orow + (vi - NSV) * EPV, r);
        }
    }
}

// Linear mode, seqlen 1, state_len == W-1 (H <= 4): a lane owns NS dwords of
// x (CPL channels each: 2 bf16/fp16, 1 fp32; dwords lane, lane + 64, ...) and
// reads their H-dword state spans directly, one dword-vector load per span;
// consecutive lanes hold consecutive spans, so each load instruction covers
// 64 * 4H contiguous bytes. No LDS and no shuffle between the loads, the
// arithmetic and the stores. A wavefront takes 64 * NS * CPL channels of BPW
// batch entries, a workgroup WPG consecutive channel groups of the same
// entries (grid: workgroups along the channels x batch-entry groups); x first, then
// the BPW pool indices (scalar loads) behind a scheduling fence, then the
// state spans, then the weights and bias (cache-resident), all before any
// arithmetic.
template <typename T, int W, int BPW, int NS, int WPG, bool SILU, bool HAS_BIAS, bool HAS_IDX>
__global__ void __launch_bounds__(64 * WPG) update_dir(const LinArgs<T> a) {
    constexpr int H = W - 1;
    constexpr int CPL = 4 / (int)sizeof(T);
    static_assert(H >= 1 && H <= 4, "one dword vector of state per span");
    const int lane = threadIdx.x & 63;
    const uint32_t grp = blockIdx.x * WPG + (threadIdx.x >> 6);  // channel group of this wavefront
    uint32_t c[NS];
    bool on[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        const uint32_t cu = (grp * (64 * NS) + 64 * u + lane) * CPL;
        on[u] = cu < a.dim;
        c[u] = on[u] ? cu : 0;  // lanes past the end read channel 0 and store nothing
    }
    const uint32_t b0 = blockIdx.y * BPW;
    const uint32_t nb = a.nbatch;
    // the first entry's index address, formed (in scalar registers) before the x loads
    const int32_t* ip = HAS_IDX ? a.idx + b0 : nullptr;
    if constexpr (HAS_IDX) asm volatile("" ::"s"(ip));
    uint32_t xd[BPW][NS];
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
        const uint32_t b = min(b0 + q, nb - 1);
#pragma unroll
        for (int u = 0; u < NS; ++u)
            xd[q][u] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(a.x + (size_t)b * a.x_row + c[u]));
    }
    // the pool indices (scalar loads) after the index-free x loads; the fence
    // keeps the compiler from hoisting them and their wait above those
    __builtin_amdgcn_sched_barrier(0);
    int32_t row[BPW];
    if constexpr (HAS_IDX) {
        int32_t r[BPW];
        // one scalar load for a pair when both entries exist and the pair is 8-byte aligned
        if (BPW == 2 && b0 + 1 < nb && (reinterpret_cast<uintptr_t>(ip) & 7u) == 0) {
            const uint64_t two = *(const __attribute__((address_space(4))) uint64_t*)reinterpret_cast<uintptr_t>(ip);
            r[0] = (int32_t)(uint32_t)two;
            r[BPW - 1] = (int32_t)(uint32_t)(two >> 32);
        } else {
#pragma unroll
            for (int q = 0; q < BPW; ++q) r[q] = ld_uniform(ip + (b0 + q < nb ? q : 0));
        }
#pragma unroll
        for (int q = 0; q < BPW; ++q)
            row[q] = (r[q] < 0 || r[q] >= a.state_rows) ? -1 : r[q];  // padding (any negative) or out of the pool
    } else {
        // without indices, entry b uses row b; an entry past the batch (odd
        // batch, last wavefront) reads row nb-1, in bounds, and stores nothing
#pragma unroll
        for (int q = 0; q < BPW; ++q) row[q] = (int32_t)min(b0 + q, nb - 1);
    }
    uint32_t st[BPW][NS][H];
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
        const T* srow = a.conv_state + (size_t)(row[q] >= 0 ? row[q] : 0) * a.state_row;
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const uint32_t* sp = reinterpret_cast<const uint32_t*>(srow + (size_t)c[u] * H);
#pragma unroll
            for (int i = 0; i < H; ++i) st[q][u][i] = __builtin_nontemporal_load(&sp[i]);
        }
    }
    // weights and bias (cache-resident) after the state loads: they arrive
    // with the state instead of holding the state loads' issue back
    uint32_t wd[NS][W], bd[NS];  // CPL * W weights and CPL biases per span, raw
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(a.weight + (size_t)c[u] * W);
#pragma unroll
        for (int k = 0; k < W; ++k) wd[u][k] = wp[k];
        bd[u] = HAS_BIAS ? *reinterpret_cast<const uint32_t*>(a.bias + c[u]) : 0u;
    }
    __builtin_amdgcn_sched_barrier(0);  // every load is issued before any arithmetic
    auto elem = [&](const uint32_t* d, int n) -> uint32_t {
        if constexpr (CPL == 1) return d[n];
        else return (n & 1) ? (d[n >> 1] >> 16) : (d[n >> 1] & 0xffffu);
    };
    auto as_f32 = [&](uint32_t bits) -> float {
        if constexpr (CPL == 1) return __uint_as_float(bits);
        else return to_f32(T{(uint16_t)bits});
    };
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            uint32_t sraw[CPL * H], nraw[CPL * H];
#pragma unroll
            for (int n = 0; n < CPL * H; ++n) sraw[n] = elem(st[q][u], n);
            float o[CPL];
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
                const uint32_t xb = elem(&xd[q][u], e);
                float win[W], w[W];
#pragma unroll
                for (int i = 0; i < H; ++i) win[i] = as_f32(sraw[e * H + i]);
                win[H] = as_f32(xb);
#pragma unroll
                for (int k = 0; k < W; ++k) w[k] = as_f32(elem(wd[u], e * W + k));
                const float bias = HAS_BIAS ? as_f32(elem(&bd[u], e)) : 0.0f;
                float acc = conv_taps<W>(bias, w, win);
                if constexpr (SILU) acc = silu(acc);
                o[e] = acc;
#pragma unroll
                for (int i = 0; i < H; ++i) nraw[e * H + i] = i + 1 < H ? sraw[e * H + i + 1] : xb;
            }
            uint32_t od;
            if constexpr (CPL == 1) od = __float_as_uint(o[0]);
            else od = pack2<T>(o[0], o[1]);
            if (row[q] < 0) od = 0u;  // padding entry: zero output, state untouched
            if (on[u] && b0 + q < nb) {  // (an entry past the batch computed on clamped data)
                __builtin_nontemporal_store(od, reinterpret_cast<uint32_t*>(a.out + (size_t)(b0 + q) * a.out_row + c[u]));
                if (row[q] >= 0) {
                    uint32_t* sp = reinterpret_cast<uint32_t*>(a.conv_state + (size_t)row[q] * a.state_row +
                                                               (size_t)c[u] * H);
#pragma unroll
                    for (int i = 0; i < H; ++i)
                        __builtin_nontemporal_store(CPL == 1 ? nraw[i] : (nraw[2 * i] | (nraw[2 * i + 1] << 16)), &sp[i]);
                }
            }
        }
    }
}

// Circular mode with at most LMAX new tokens: one thread per (b, c), lanes on
// adjacent channels. Every load (W-1 history values, the new tokens) is
// issued before any arithmetic or store, so each lane keeps all of its
// scattered state accesses in flight at once.
template <typename T, int W, bool SILU, int LMAX>
__global__ void __launch_bounds__(256) update_circ(const UpdArgs a) {
    constexpr int H = W - 1;
    const cc1d_update_params& p = a.p;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n_items) return;
    const int64_t c = idx % p.dim;
    const int64_t b = idx / p.dim;
    const int Ls = (int)p.seqlen;
    const int64_t S = p.state_len;
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];
    const int64_t row = state_row(p, b);
    if (row < 0) {
#pragma unroll
        for (int i = 0; i < LMAX; ++i)
            if (i < Ls) st(orow, i * p.out_stride[2], 0.0f);
        return;
    }
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    T* __restrict__ sr = static_cast<T*>(p.conv_state) + row * p.conv_state_stride[0] + c * p.conv_state_stride[1];
    const int64_t ss = p.conv_state_stride[2];
    int64_t cs = (int64_t)p.cache_seqlens[b] % S;
    if (cs < 0) cs += S;  // floored modulo (torch.remainder)
    int64_t head = cs - H;
    if (head < 0) head += S;

    T hist[H > 0 ? H : 1];
    T xv[LMAX];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        int64_t pos = head + i;
        if (pos >= S) pos -= S;
        hist[i] = sr[pos * ss];
    }
#pragma unroll
    for (int i = 0; i < LMAX; ++i)
        if (i < Ls) xv[i] = xr[i * p.x_stride[2]];

    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        w[k] = ld(static_cast<const T*>(p.weight), c * p.weight_stride[0] + k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), c * p.bias_stride) : 0.0f;

    float win[W];
#pragma unroll
    for (int i = 0; i < H; ++i) win[i] = to_f32(hist[i]);
    int64_t wpos = cs;
#pragma unroll
    for (int i = 0; i < LMAX; ++i) {
        if (i < Ls) {
            sr[wpos * ss] = xv[i];
            if (++wpos >= S) wpos -= S;
            win[H] = to_f32(xv[i]);
            float acc = conv_taps<W>(bias, w, win);
            if constexpr (SILU) acc = silu(acc);
            st(orow, i * p.out_stride[2], acc);
#pragma unroll
            for (int k = 0; k < H; ++k) win[k] = win[k + 1];
        }
    }
}

// Replace element e (compile-time after unrolling) of a 16-byte vector by
// the raw bits of a T.
template <typename T> __device__ __forceinline__ void vset_raw(u32x4& v, int e, uint32_t bits) {
    if constexpr (sizeof(T) == 4) {
        v[e] = bits;
    } else {
        const uint32_t d = v[e >> 1];
        v[e >> 1] = (e & 1) ? ((d & 0x0000ffffu) | (bits << 16)) : ((d & 0xffff0000u) | (bits & 0xffffu));
    }
}
template <typename T> __device__ __forceinline__ uint32_t raw_bits(const T* p) {
    if constexpr (sizeof(T) == 4) return *reinterpret_cast<const uint32_t*>(p);
    else return *reinterpret_cast<const uint16_t*>(p);
}

// Circular mode on contiguous, 16-byte aligned state lines whose length is a
// multiple of the 16-byte chunk (EPV elements), with a window of W-1 history
// plus Ls new positions that spans at most two chunks: ka and the chunk kb
// after it. Two adjacent lanes per (b, c): the lead lane reads chunk ka, its
// partner chunk kb -- one 32-byte access when kb follows ka in memory -- and
// they swap the chunks, so both hold the window. The window starts at offset
// O (compile-time) inside ka, so every element access is a register access.
// Both lanes write the new tokens into their copies and compute the outputs;
// the lead lane writes the outputs and stores chunk ka back whole, the
// partner stores chunk kb when the window reaches into it (the other
// positions of a chunk are written back unchanged; only this pair touches
// this state line).
template <typename T, int W, bool SILU, bool DW, int O>
__device__ __forceinline__ void update_circ_chunks(const cc1d_update_params& p, uint32_t b, uint32_t c, T* sl,
                                                   int32_t ka, int32_t kb, int Ls, const uint32_t* xb,
                                                   const float* w, float bias, u32x4 va, u32x4 vb, bool lead) {
    constexpr int H = W - 1;
    constexpr int EPV = elems16<T>::value;
    constexpr int LMAX = EPV + 1 - H;  // most new tokens a two-chunk window holds
    const bool cross = O + H + Ls > EPV;

    float win[W];
#pragma unroll
    for (int i = 0; i < H; ++i) win[i] = (O + i < EPV) ? vget<T>(va, O + i) : vget<T>(vb, O + i - EPV);
    T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];
    float o[LMAX];
#pragma unroll
    for (int i = 0; i < LMAX; ++i) {
        o[i] = 0.0f;
        if (i < Ls) {
            const int q = O + H + i;  // window position of new token i
            if (q < EPV) vset_raw<T>(va, q, xb[i]);
            else vset_raw<T>(vb, q - EPV, xb[i]);
            u32x4 one = vzero();
            vset_raw<T>(one, 0, xb[i]);
            win[H] = vget<T>(one, 0);
            float acc = conv_taps<W>(bias, w, win);
            if constexpr (SILU) acc = silu(acc);
            o[i] = acc;
            if constexpr (!DW) {
                if (lead) st(orow, i * p.out_stride[2], acc);
            }
#pragma unroll
            for (int k = 0; k < H; ++k) win[k] = win[k + 1];
        }
    }
    if constexpr (DW) {  // the Ls outputs as whole dwords
        constexpr int PER = 4 / (int)sizeof(T);
#pragma unroll
        for (int d = 0; d < (LMAX + PER - 1) / PER; ++d) {
            if (lead && d * PER < Ls) {
                uint32_t v;
                if constexpr (PER == 1) v = __float_as_uint(o[d]);
                else v = pack2<T>(o[2 * d], o[2 * d + 1 < LMAX ? 2 * d + 1 : 0]);
                __builtin_nontemporal_store(v, reinterpret_cast<uint32_t*>(orow) + d);
            }
        }
    }
    if (lead) vstore(sl + ka * EPV, va);
    else if (cross) vstore(sl + kb * EPV, vb);
}

// DPP quad_perm [1, 0, 3, 2]: each lane reads its pair partner (lane ^ 1)
constexpr int kQuadSwapPairs = 1 | (0 << 2) | (3 << 4) | (2 << 6);

template <typename T, int W, bool SILU, bool DW>
__global__ void __launch_bounds__(256) update_circ_vec(const UpdArgs a) {
    constexpr int H = W - 1;
    constexpr int EPV = elems16<T>::value;
    constexpr int LMAX = EPV + 1 - H;
    static_assert(LMAX >= 1, "window must fit in two chunks");
    const cc1d_update_params& p = a.p;
    const uint32_t tid = blockIdx.x * 256 + threadIdx.x;
    if (tid >= (uint32_t)a.n_items) return;  // n_items is even: a pair leaves together
    const uint32_t idx = tid >> 1;           // (b, c)
    const bool lead = (tid & 1u) == 0;
    const uint32_t D = (uint32_t)p.dim;
    const uint32_t b = idx / D;
    const uint32_t c = idx - b * D;
    const int Ls = (int)p.seqlen;
    // inputs that do not depend on the state row first, so their loads overlap
    // the index / cache_seqlens reads the state addresses wait for
    const T* __restrict__ xr = static_cast<const T*>(p.x) + b * p.x_stride[0] + c * p.x_stride[1];
    uint32_t xb[LMAX];
    if constexpr (DW) {  // the Ls tokens as whole dwords
        constexpr int PER = 4 / (int)sizeof(T);
#pragma unroll
        for (int d = 0; d < (LMAX + PER - 1) / PER; ++d) {
            const uint32_t v = d * PER < Ls ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(xr) + d) : 0u;
#pragma unroll
            for (int e = 0; e < PER; ++e)
                if (d * PER + e < LMAX) xb[d * PER + e] = PER == 1 ? v : ((v >> (16 * e)) & 0xffffu);
        }
    } else {
#pragma unroll
        for (int i = 0; i < LMAX; ++i) xb[i] = i < Ls ? raw_bits(xr + i * p.x_stride[2]) : 0u;
    }
    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        w[k] = ld(static_cast<const T*>(p.weight), (int64_t)c * p.weight_stride[0] + k * p.weight_stride[1]);
    const float bias = p.bias ? ld(static_cast<const T*>(p.bias), (int64_t)c * p.bias_stride) : 0.0f;

    const int64_t row = state_row(p, b);
    if (row < 0) {  // the same for both lanes of a pair
        if (lead) {
            T* __restrict__ orow = static_cast<T*>(p.out) + b * p.out_stride[0] + c * p.out_stride[1];
            for (int i = 0; i < Ls; ++i) st(orow, i * p.out_stride[2], 0.0f);
        }
        return;
    }
    const int32_t S = (int32_t)p.state_len;
    T* __restrict__ sl = static_cast<T*>(p.conv_state) + row * p.conv_state_stride[0] + c * p.conv_state_stride[1];
    int32_t cs = p.cache_seqlens[b] % S;
    if (cs < 0) cs += S;  // floored modulo (torch.remainder)
    int32_t p0 = cs - H;  // first window position
    if (p0 < 0) p0 += S;
    const int32_t ka = p0 / EPV;
    const int32_t kb = ka + 1 < S / EPV ? ka + 1 : 0;  // the chunk after ka, cyclically
    // each lane of the pair reads one chunk; a quad-permute DPP move (lanes
    // 0<->1, 2<->3) hands each the other's
    const u32x4 mine = vload(sl + (lead ? ka : kb) * EPV);
    u32x4 other;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        other[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine[i], kQuadSwapPairs, 0xf, 0xf, false);
    const u32x4 va = lead ? mine : other;
    const u32x4 vb = lead ? other : mine;
    switch (p0 % EPV) {
        case 0: update_circ_chunks<T, W, SILU, DW, 0>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
        case 1: update_circ_chunks<T, W, SILU, DW, 1>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
        case 2: update_circ_chunks<T, W, SILU, DW, 2>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
        case 3: update_circ_chunks<T, W, SILU, DW, 3>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
        default:
            if constexpr (EPV == 8) {
                switch (p0 % EPV) {
                    case 4: update_circ_chunks<T, W, SILU, DW, 4>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
                    case 5: update_circ_chunks<T, W, SILU, DW, 5>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
                    case 6: update_circ_chunks<T, W, SILU, DW, 6>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
                    default: update_circ_chunks<T, W, SILU, DW, 7>(p, b, c, sl, ka, kb, Ls, xb, w, bias, va, vb, lead); break;
                }
            }
            break;
    }
}

namespace {

// update_lin: 16-byte vectors per lane (each wavefront covers 16 * EPV * kLinNV
// channels). C4a (256 x 5120 bf16, W4): 1 -> 7.58 us, 2 -> 7.12 us, 4 -> 7.50 us.
constexpr int kLinNV = 2;
// update_dir: batch entries per wavefront and dwords of x per lane. C4a (A/B
// on one box, update_lin 7.14 us): 2 x 1 -> 6.97 us; 1 x 1 7.06; 4 x 1 7.03;
// 2 x 2 7.38; 1 x 2 7.15; 1 x 4 7.48; 4 x 2 7.80. Wider contiguous spans per
// lane (2 or 4 dwords of x, 6 or 12 of state, so that one load instruction no
// longer covers contiguous bytes): 7.50 / 8.05 us. Without SiLU, or with the
// weights and bias replaced by constants, 2 x 1 measures the same 6.97-7.05 us:
// what is left is the access pattern (a copy that moves the same bytes as
// 16-byte vectors, one x and three state vectors per lane, takes ~0.4 us less).
constexpr int kDirBPW = 2;
constexpr int kDirNS = 1;
// update_dir: wavefronts (consecutive channel groups) per workgroup. C4a, with
// 2 batch entries per wavefront (one A/B session): 1 -> 6.96-6.97 us, 2 ->
// 6.81-6.82, 4 -> 6.76-6.78, 8 -> 7.07-7.08; 1 entry x 4 wavefronts 7.55,
// 4 entries x 4 wavefronts 7.08. The scattered-row copy does not gain from
// wider workgroups (6.50 us with 1, 6.53 with 2, 4 or 5 wavefronts).
constexpr int kDirWPG = 4;

template <typename T>
bool lin_ok(const cc1d_update_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    const int64_t H = p.width - 1;
    if (p.cache_seqlens != nullptr || p.seqlen != 1 || p.state_len != H) return false;
    if (p.dim % EPV != 0) return false;
    if (p.x_stride[1] != 1 || p.out_stride[1] != 1) return false;
    if (p.x_stride[0] % EPV || p.out_stride[0] % EPV) return false;
    if (p.conv_state_stride[2] != 1 || p.conv_state_stride[1] != H || p.conv_state_stride[0] % EPV) return false;
    if (p.weight_stride[1] != 1 || p.weight_stride[0] != p.width) return false;
    if (p.bias != nullptr && (p.bias_stride != 1 || (reinterpret_cast<uintptr_t>(p.bias) & 3u))) return false;
    if (!aligned16(p.x) || !aligned16(p.out) || !aligned16(p.conv_state) ||
        (reinterpret_cast<uintptr_t>(p.weight) & 3u))
        return false;
    // 32-bit channel indices and row strides, a grid of (groups, batch) blocks; size_t offsets
    const int64_t lim = (int64_t)1 << 31;
    if (p.dim >= lim || p.batch > 65535 || p.state_rows >= lim) return false;
    if (p.x_stride[0] >= lim || p.out_stride[0] >= lim || p.conv_state_stride[0] >= lim) return false;
    if (p.x_stride[0] < 0 || p.out_stride[0] < 0 || p.conv_state_stride[0] < 0) return false;
    return true;
}

// chunked circular mode: contiguous 16-byte aligned state lines of at least
// two whole chunks, a window of W-1 + seqlen positions within two chunks
template <typename T>
bool circ_vec_ok(const cc1d_update_params& p) {
    constexpr int64_t EPV = elems16<T>::value;
    if (p.cache_seqlens == nullptr || p.seqlen < 1) return false;
    if (p.width - 1 + p.seqlen > EPV + 1) return false;
    // two distinct chunks per line, so a window never wraps onto itself
    if (p.state_len % EPV != 0 || p.state_len < 2 * EPV) return false;
    if (p.conv_state_stride[2] != 1 || p.conv_state_stride[1] % EPV || p.conv_state_stride[0] % EPV) return false;
    if (!aligned16(p.conv_state)) return false;
    if (2 * p.batch * p.dim >= ((int64_t)1 << 31) || p.state_len >= ((int64_t)1 << 31)) return false;
    return true;
}

// tokens of x and out contiguous, a whole number of dwords, dword-aligned rows
template <typename T>
bool circ_dwords_ok(const cc1d_update_params& p) {
    const int64_t e = (int64_t)sizeof(T);
    if (p.x_stride[2] != 1 || p.out_stride[2] != 1 || (p.seqlen * e) % 4) return false;
    if (((p.x_stride[0] | p.x_stride[1] | p.out_stride[0] | p.out_stride[1]) * e) % 4) return false;
    return ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.out)) & 3u) == 0;
}

}  // namespace

int launch_update(const cc1d_update_params& p, hipStream_t stream) {
    return with_dtype(p.dtype, [&](auto tag) {
        using T = decltype(tag);
        constexpr int64_t EPV = elems16<T>::value;
        return with_width(p.width, [&](auto wc) {
            constexpr int W = decltype(wc)::value;
            return with_flag(p.apply_silu != 0, [&](auto sc) {
                constexpr bool SILU = decltype(sc)::value;
                UpdArgs a;
                a.p = p;
                if (lin_ok<T>(p)) {
                    LinArgs<T> la;
                    la.x = static_cast<const T*>(p.x);
                    la.weight = static_cast<const T*>(p.weight);
                    la.bias = static_cast<const T*>(p.bias);
                    la.conv_state = static_cast<T*>(p.conv_state);
                    la.idx = p.conv_state_indices;
                    la.out = static_cast<T*>(p.out);
                    la.x_row = (uint32_t)p.x_stride[0];
                    la.out_row = (uint32_t)p.out_stride[0];
                    la.state_row = (uint32_t)p.conv_state_stride[0];
                    la.dim = (uint32_t)p.dim;
                    la.state_rows = (int32_t)p.state_rows;
                    la.nbatch = (uint32_t)p.batch;
                    if constexpr (W - 1 <= 4) {
                        constexpr int CPL = 4 / (int)sizeof(T);
                        const dim3 gd((unsigned)ceil_div(ceil_div(p.dim, 64 * kDirNS * CPL), kDirWPG),
                                      (unsigned)ceil_div(p.batch, kDirBPW));
                        return with_flag(p.bias != nullptr, [&](auto hb) {
                            return with_flag(p.conv_state_indices != nullptr, [&](auto hi) {
                                return launch(update_dir<T, W, kDirBPW, kDirNS, kDirWPG, SILU, decltype(hb)::value,
                                                         decltype(hi)::value>,
                                              gd, dim3(64 * kDirWPG), stream, la);
                            });
                        });
                    }
                    // grid: channel groups x batch entries (no division in the kernel)
                    const dim3 grid((unsigned)ceil_div(p.dim, 16 * EPV * kLinNV), (unsigned)p.batch);
                    return with_flag(p.bias != nullptr, [&](auto hb) {
                        return with_flag(p.conv_state_indices != nullptr, [&](auto hi) {
                            return launch(update_lin<T, W, kLinNV, SILU, decltype(hb)::value, decltype(hi)::value>,
                                          grid, dim3(64), stream, la);
                        });
                    });
                }
                a.n_items = p.batch * p.dim;
                const dim3 grid((unsigned)ceil_div(a.n_items, 256));
                if constexpr (W - 1 <= EPV) {
                    if (circ_vec_ok<T>(p)) {
                        a.n_items = 2 * p.batch * p.dim;  // two lanes per (b, c)
                        return with_flag(circ_dwords_ok<T>(p), [&](auto dc) {
                            return launch(update_circ_vec<T, W, SILU, decltype(dc)::value>,
                                          dim3((unsigned)ceil_div(a.n_items, 256)), dim3(256), stream, a);
                        });
                    }
                }
                if (p.cache_seqlens != nullptr && p.seqlen <= 8) {
                    return launch(update_circ<T, W, SILU, 8>, grid, dim3(256), stream, a);
                }
                return with_flag(p.cache_seqlens != nullptr, [&](auto cc) {
                    constexpr bool CIRC = decltype(cc)::value;
                    return launch(update_generic<T, W, SILU, CIRC>, grid, dim3(256), stream, a);
                });
            });
        });
    });
}

}  // namespace cc1d
