// cc1d_device.hpp -- device helpers shared by the gfx950 causal conv1d kernels.
//
// Storage types are tag structs around the raw bits so that every conversion
// is explicit: bf16/fp16 widen exactly to fp32 and narrow with one
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32 / v_cvt_f16_f32 on
// gfx950). Rows move through HBM as 16-byte vectors (global_load_dwordx4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cc1d_fastdiv.hpp"

namespace cc1d {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct f16 { uint16_t bits; };
struct bf16 { uint16_t bits; };

template <typename T> struct elems16 { static constexpr int value = 16 / (int)sizeof(T); };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return __uint_as_float((uint32_t)v.bits << 16); }
__device__ __forceinline__ float to_f32(f16 v) { return (float)__builtin_bit_cast(_Float16, v.bits); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) {
    return bf16{__builtin_bit_cast(uint16_t, (__bf16)v)};
}
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) {
    return f16{__builtin_bit_cast(uint16_t, (_Float16)v)};
}

// Two fp32 values narrowed into one dword, a in the low half: one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 (RNE, the same rounding as from_f32).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Round-trip through the storage dtype (what a store followed by a load gives).
template <typename T> __device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

// Element e (compile-time after unrolling) of a 16-byte vector, widened to fp32.
template <typename T> __device__ __forceinline__ float vget(const u32x4& v, int e);
template <> __device__ __forceinline__ float vget<float>(const u32x4& v, int e) { return __uint_as_float(v[e]); }
template <> __device__ __forceinline__ float vget<bf16>(const u32x4& v, int e) {
    const uint32_t d = v[e >> 1];
    return (e & 1) ? __uint_as_float(d & 0xffff0000u) : __uint_as_float(d << 16);
}
template <> __device__ __forceinline__ float vget<f16>(const u32x4& v, int e) {
    const uint32_t d = v[e >> 1];
    const uint16_t h = (e & 1) ? (uint16_t)(d >> 16) : (uint16_t)(d & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, h);
}

// Pack EPV fp32 values into one 16-byte vector of T (one RNE rounding each).
template <typename T> __device__ __forceinline__ u32x4 vpack(const float* f);
template <> __device__ __forceinline__ u32x4 vpack<float>(const float* f) {
    u32x4 r;
    r[0] = __float_as_uint(f[0]); r[1] = __float_as_uint(f[1]);
    r[2] = __float_as_uint(f[2]); r[3] = __float_as_uint(f[3]);
    return r;
}
template <> __device__ __forceinline__ u32x4 vpack<bf16>(const float* f) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = pack2<bf16>(f[2 * d], f[2 * d + 1]);
    return r;
}
template <> __device__ __forceinline__ u32x4 vpack<f16>(const float* f) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) r[d] = pack2<f16>(f[2 * d], f[2 * d + 1]);
    return r;
}

__device__ __forceinline__ u32x4 vzero() { u32x4 z = {0u, 0u, 0u, 0u}; return z; }

template <typename T> __device__ __forceinline__ u32x4 vload(const T* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
template <typename T> __device__ __forceinline__ void vstore(T* p, const u32x4& v) {
    *reinterpret_cast<u32x4*>(p) = v;
}

// Streaming (non-temporal) 16-byte accesses for data touched exactly once:
// global_load/store_dwordx4 ... nt, so the stream does not displace reused
// lines (weights, seq_idx, halos) from L2 / the Infinity Cache.
template <typename T> __device__ __forceinline__ u32x4 vload_nt(const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
template <typename T> __device__ __forceinline__ void vstore_nt(T* p, const u32x4& v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// N consecutive elements of T held as raw dwords, N * sizeof(T) in {4, 8, 16}
// (one global_load / store of 1, 2 or 4 dwords per lane). Element indices
// are compile-time after unrolling.
template <typename T, int N> struct Lanes {
    static constexpr int ND = N * (int)sizeof(T) / 4;
    static_assert(ND == 1 || ND == 2 || ND == 4, "4, 8 or 16 bytes per lane");
    uint32_t d[ND];

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < ND; ++i) d[i] = 0u;
    }
    template <bool NT> __device__ __forceinline__ void load(const T* p) {
        if constexpr (ND == 4) {
            const u32x4 v = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p))
                               : *reinterpret_cast<const u32x4*>(p);
            d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
        } else if constexpr (ND == 2) {
            const u32x2 v = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p))
                               : *reinterpret_cast<const u32x2*>(p);
            d[0] = v[0]; d[1] = v[1];
        } else {
            d[0] = NT ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p))
                      : *reinterpret_cast<const uint32_t*>(p);
        }
    }
    template <bool NT> __device__ __forceinline__ void store(T* p) const {
        if constexpr (ND == 4) {
            const u32x4 v = {d[0], d[1], d[2], d[3]};
            if (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
            else *reinterpret_cast<u32x4*>(p) = v;
        } else if constexpr (ND == 2) {
            const u32x2 v = {d[0], d[1]};
            if (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
            else *reinterpret_cast<u32x2*>(p) = v;
        } else {
            if (NT) __builtin_nontemporal_store(d[0], reinterpret_cast<uint32_t*>(p));
            else *reinterpret_cast<uint32_t*>(p) = d[0];
        }
    }
    __device__ __forceinline__ float get(int e) const {
        if constexpr (sizeof(T) == 4) {
            return __uint_as_float(d[e]);
        } else {
            const uint32_t w = d[e >> 1];
            if constexpr (__is_same(T, bf16)) {
                return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
            } else {
                const uint16_t h = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
                return (float)__builtin_bit_cast(_Float16, h);
            }
        }
    }
    __device__ __forceinline__ void set(const float* f) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int i = 0; i < ND; ++i) d[i] = __float_as_uint(f[i]);
        } else {
#pragma unroll
            for (int i = 0; i < ND; ++i) d[i] = pack2<T>(f[2 * i], f[2 * i + 1]);
        }
    }
};

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }

// Reads of wave-uniform addresses through the scalar data cache (constant
// address space): for data that no wavefront writes during the kernel, such
// as weights, bias and halo vectors of read-only inputs. Their completion is
// tracked by lgkmcnt, so waiting for them never waits for the wavefront's
// outstanding vector-memory reads.
typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;
typedef const __attribute__((address_space(4))) u32x4* const_u32x4_ptr;

// Element at p (wave-uniform), widened to fp32: reads the aligned dword holding it.
template <typename T> __device__ __forceinline__ float ld_uniform(const T* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t d = *(const_u32_ptr)(a & ~(uintptr_t)3);
    if constexpr (sizeof(T) == 4) {
        return __uint_as_float(d);
    } else {
        const uint16_t h = (a & 2) ? (uint16_t)(d >> 16) : (uint16_t)(d & 0xffffu);
        return to_f32(T{h});
    }
}
__device__ __forceinline__ int32_t ld_uniform(const int32_t* p) {
    return (int32_t)*(const_u32_ptr)reinterpret_cast<uintptr_t>(p);
}
// 16-byte vector at the wave-uniform, 16-byte aligned address p.
template <typename T> __device__ __forceinline__ u32x4 vload_uniform(const T* p) {
    return *(const_u32x4_ptr)reinterpret_cast<uintptr_t>(p);
}
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }

// Dword d of a 16-byte vector of T: the bits of its elements e < n (all of
// them for n >= EPV, none for n <= 0).
template <typename T> __device__ __forceinline__ uint32_t lead_mask(int d, int32_t n) {
    if constexpr (sizeof(T) == 4) return d < n ? ~0u : 0u;
    else return 2 * d + 1 < n ? ~0u : (2 * d < n ? 0xffffu : 0u);
}
// Storage bits of an fp32 value that T represents exactly.
template <typename T> __device__ __forceinline__ uint32_t tbits(float v) {
    if constexpr (sizeof(T) == 4) return __float_as_uint(v);
    else return from_f32<T>(v).bits;
}
// Store element e of the packed vector v at p (its raw bits: no rounding).
template <typename T> __device__ __forceinline__ void st_elem(T* p, const u32x4& v, int e) {
    if constexpr (sizeof(T) == 4) *reinterpret_cast<uint32_t*>(p) = v[e];
    else *reinterpret_cast<uint16_t*>(p) = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
}

// a[k] for a runtime k (0 outside [0, N)), as a chain of selects: a register
// array indexed at run time would be placed in scratch memory
template <int N> __device__ __forceinline__ float pick(const float* a, int k) {
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) r = (i == k) ? a[i] : r;
    return r;
}

// Wavefront-uniform value (lets the compiler keep it in an SGPR).
__device__ __forceinline__ uint32_t uniform32(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uniform_f32(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ int64_t uniform(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
// A per-lane value the compiler can neither see through nor move: address
// arithmetic of a rarely taken branch that uses it stays inside the branch
// instead of being hoisted out of the loop around it (where it would hold
// registers for the whole loop).
__device__ __forceinline__ int32_t opaque(int32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// The N (4 or 8) ids of row positions pos .. pos + N - 1 of one seq_idx row
// (sr, L ids, unit stride; -1 outside [0, L)), read as the N/4 + 1 aligned
// 16-byte vectors that cover them (ids_load) and shifted into place
// (ids_shift): r = the first id's offset in its vector (the same for every
// lane), a0 = sr's own offset in its vector. MASK: some position may lie
// outside the row; a lane with none inside loads nothing, and a vector that
// holds none of the row's ids reads the row's first vector instead, as does
// the last one when r == 0 (not needed then), so every access stays inside
// the row's allocation. A kernel issues every vector's loads before the
// first shift: a shift right behind its loads waits for them, before the
// next vector's loads are issued.
template <int N> struct IdsRaw {
    u32x4 v[N / 4 + 1];
};

template <int N, bool MASK>
__device__ __forceinline__ void ids_load(const int32_t* sr, int32_t L, int32_t pos, int r, int a0, IdsRaw<N>& raw) {
    static_assert(N == 4 || N == 8, "one or two 16-byte vectors");
    constexpr int NV = N / 4 + 1;
    const int32_t q0 = pos - r;  // first row position of the first vector (16-byte aligned)
    if (!MASK || (pos + N > 0 && pos < L)) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            int32_t q = q0 + 4 * v;
            if (v == NV - 1) q = r != 0 ? q : q0;
            if constexpr (MASK) q = (q + 3 >= 0 && q < L) ? q : -a0;
            raw.v[v] = *reinterpret_cast<const u32x4*>(sr + q);
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) raw.v[v] = vzero();  // masked to -1 by ids_shift
    }
}

// The shift is two levels of v_perm_b32 (one dword of two, by the bits of
// r): selects on a scalar r became branches, each waiting for its loads, and
// selects on a vector-register r an indexed copy through scratch memory.
template <int N, bool MASK>
__device__ __forceinline__ void ids_shift(const IdsRaw<N>& raw, int32_t L, int32_t pos, int r, int32_t* out) {
    uint32_t c[N + 4];
#pragma unroll
    for (int v = 0; v < N / 4 + 1; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) c[4 * v + i] = raw.v[v][i];
    // byte selectors of v_perm_b32(hi, lo, sel): 0x07060504 picks hi, 0x03020100 lo
    const uint32_t s2 = (r & 2) ? 0x07060504u : 0x03020100u;
    const uint32_t s1 = (r & 1) ? 0x07060504u : 0x03020100u;
    uint32_t t[N + 2];
#pragma unroll
    for (int e = 0; e < N + 2; ++e) t[e] = __builtin_amdgcn_perm(c[e + 2], c[e], s2);
#pragma unroll
    for (int e = 0; e < N; ++e) {
        out[e] = (int32_t)__builtin_amdgcn_perm(t[e + 1], t[e], s1);
        if constexpr (MASK) out[e] = (pos + e >= 0 && pos + e < L) ? out[e] : -1;
    }
}

// SiLU = x * sigmoid(x), as x * rcp(1 + exp(-x)) in fp32.
__device__ __forceinline__ float silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// d silu / d x = s * (1 + x * (1 - s)), s = sigmoid(x).
__device__ __forceinline__ float silu_grad(float x) {
    const float s = __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    return s * (1.0f + x * (1.0f - s));
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// g * silu'(p) given q = -log2(e) * p (so exp(-p) = exp2(q)):
//   s = 1 / (1 + exp2(q));  g * s * (1 + p * (1 - s)) = gs + (gs * q) * (-ln2 * (1 - s))
// Five VALU operations plus exp2 and rcp.
__device__ __forceinline__ float silu_bwd_q(float g, float q) {
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(q));
    const float gs = g * s;
    return __builtin_fmaf(gs * q, __builtin_fmaf(s, kLn2, -kLn2), gs);
}

// Causal taps: bias + sum_k w[k] * win[k], fp32 fma in k order. The forward
// and the decode update both use this, so a decode loop reproduces the full
// forward bit for bit.
template <int W>
__device__ __forceinline__ float conv_taps(float bias, const float* w, const float* win) {
    float acc = bias;
#pragma unroll
    for (int k = 0; k < W; ++k) acc = __builtin_fmaf(w[k], win[k], acc);
    return acc;
}

// As conv_taps, keeping tap k only when ids[k] equals the current id ids[W-1].
template <int W>
__device__ __forceinline__ float conv_taps_gated(float bias, const float* w, const float* win,
                                                 const int32_t* ids) {
    float acc = bias;
    const int32_t cur = ids[W - 1];
#pragma unroll
    for (int k = 0; k < W; ++k)
        if (ids[k] == cur) acc = __builtin_fmaf(w[k], win[k], acc);
    return acc;
}

// Value of `v` held by lane `src` of this wavefront (ds_bpermute_b32).
__device__ __forceinline__ uint32_t lane_get(uint32_t v, int src) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
}
__device__ __forceinline__ float lane_get(float v, int src) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}
__device__ __forceinline__ int32_t lane_get(int32_t v, int src) {
    return __builtin_amdgcn_ds_bpermute(src << 2, v);
}

// DPP controls (GFX9 encoding) for the wavefront reduction below.
constexpr int kDppQuadSwap1 = 0xb1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadSwap2 = 0x4e;   // quad_perm [2, 3, 0, 1]
constexpr int kDppRowRor4 = 0x124;    // row_ror:4 (rotate within 16 lanes)
constexpr int kDppRowRor8 = 0x128;    // row_ror:8
constexpr int kDppRowBcast15 = 0x142; // row_bcast:15 (lane 15 of a row into the next row)
constexpr int kDppRowBcast31 = 0x143; // row_bcast:31 (lane 31 into rows 2 and 3)

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v) {
    // rows outside ROW_MASK receive 0 (the `old` operand), so `v + dpp` leaves them unchanged
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wavefront, returned wave-uniform (every lane
// receives it). Cross-lane moves are DPP modifiers on VALU adds -- no LDS
// round trips: sums within quads, then rows of 16, then rows 0+1 and 2+3 into
// rows 1 and 3, then rows 0+1 into rows 2 and 3; lane 63 holds the total.
// All 64 lanes must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppQuadSwap1, 0xf>(v);
    v += dpp_f32<kDppQuadSwap2, 0xf>(v);
    v += dpp_f32<kDppRowRor4, 0xf>(v);
    v += dpp_f32<kDppRowRor8, 0xf>(v);
    v += dpp_f32<kDppRowBcast15, 0xa>(v);
    v += dpp_f32<kDppRowBcast31, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

}  // namespace cc1d
