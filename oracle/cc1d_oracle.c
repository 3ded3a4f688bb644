/*
 * cc1d_oracle.c -- CPU restatement of the reference's CPU kernels for the
 * depthwise causal conv1d hot path.
 *
 * TEST INFRASTRUCTURE ONLY (checker and CPU baseline). Nothing in the
 * causal_conv1d_amd product links or calls this file.
 *
 * What it restates, loop for loop:
 *   oracle_fwd    <- fwd_kernel_cpu      src/causal_conv1d_mojo/fwd_cpu/kernel.mojo:61-119
 *   oracle_bwd    <- bwd_kernel_cpu      src/causal_conv1d_mojo/bwd_full_cpu/kernel.mojo:108-314
 *                    _cpu_dpre_at        src/causal_conv1d_mojo/bwd_full_cpu/kernel.mojo:25-105
 *   oracle_update <- update_kernel_cpu   src/causal_conv1d_mojo/update_cpu/kernel.mojo:20-141
 *   silu          <- _silu_f32           src/causal_conv1d_mojo/_silu.mojo:11-21
 *
 * Numerics: every product/sum is an fp32 IEEE operation, accumulated in the
 * reference's order (bias first, then taps k = 0..W-1); the build uses
 * -ffp-contract=off so no FMA is formed. Inputs are widened to fp32 and each
 * output is rounded once (round-to-nearest-even) to its storage dtype.
 * The reference parallelises over the B*D rows with sync_parallelize and
 * merges per-row dweight/dbias with relaxed fp32 atomics; here the rows run
 * under OpenMP and the per-row partials are merged in batch order, which is
 * one of the orders the reference's atomics can produce.
 */
#include "cc1d_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MAX_WIDTH 9

/* ---- scalar conversions (IEEE 754 binary16 / bfloat16, RNE) ------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN: keep sign, force quiet */
        return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);      /* ties to even; overflow -> inf */
    return (uint16_t)(u >> 16);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {                               /* zero / subnormal: m * 2^-24 */
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13)); /* inf / NaN */
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) { /* inf / NaN */
        if (x == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((x >> 13) & 0x1ffu);
    }
    if (x >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (x < 0x38800000u) {                       /* below 2^-14: subnormal */
        uint32_t e = x >> 23;
        int shift = 126 - (int)e;                 /* value * 2^24 = m >> shift */
        if (shift >= 25) return sign;
        uint32_t m = (x & 0x7fffffu) | 0x800000u;
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return sign | (uint16_t)r;
    }
    uint32_t r = (x - 0x38000000u) >> 13;        /* rebias 127 -> 15 */
    uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return sign | (uint16_t)r;
}

static inline float ld(const void* p, int64_t i, int dt) {
    switch (dt) {
    case 0: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    case 1: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

static inline void st(void* p, int64_t i, int dt, float v) {
    switch (dt) {
    case 0: ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
    case 1: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
    default: ((float*)p)[i] = v; break;
    }
}

/* _silu.mojo:21 -- x * recip(1 + exp(-x)) */
static inline float silu_f32(float x) { return x * (1.0f / (1.0f + expf(-x))); }

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int check_common(int dtype, int width) {
    if (dtype < 0 || dtype > 2) return 1;
    if (width < 2 || width > MAX_WIDTH) return 2;
    return 0;
}

/* ---- forward: fwd_cpu/kernel.mojo:61-119 -------------------------------- */

int oracle_fwd(int dtype, int width, int apply_silu,
               const void* x, const void* weight, const void* bias, void* out,
               int64_t batch, int64_t dim, int64_t seqlen,
               int64_t x_s0, int64_t x_s1, int64_t x_s2,
               int64_t w_s0, int64_t w_s1,
               int64_t o_s0, int64_t o_s1, int64_t o_s2,
               const int32_t* seq_idx, int64_t si_s0, int64_t si_s1,
               const void* init, int64_t is_s0, int64_t is_s1, int64_t is_s2) {
    int rc = check_common(dtype, width);
    if (rc) return rc;
    const int64_t W = width;
    const int64_t nbc = batch * dim;
#pragma omp parallel for schedule(static)
    for (int64_t bc = 0; bc < nbc; ++bc) {
        const int64_t b = bc / dim, d = bc % dim;
        float bias_v = 0.0f;
        if (bias) bias_v = ld(bias, d, dtype); /* kernel.mojo:70-71 (bias_ptr[d]) */
        float w[MAX_WIDTH];
        for (int64_t k = 0; k < W; ++k) w[k] = ld(weight, d * w_s0 + k * w_s1, dtype);
        for (int64_t t = 0; t < seqlen; ++t) {                 /* :78 */
            float pre = bias_v;
            int32_t cur = 0;
            if (seq_idx) cur = seq_idx[b * si_s0 + t * si_s1];
            for (int64_t k = 0; k < W; ++k) {                  /* :86-104 */
                const int64_t src = t + k - (W - 1);
                if (src >= 0) {
                    int include = 1;
                    if (seq_idx) include = (seq_idx[b * si_s0 + src * si_s1] == cur);
                    if (include) pre += w[k] * ld(x, b * x_s0 + d * x_s1 + src * x_s2, dtype);
                } else if (init) {
                    const int64_t ii = src + (W - 1);
                    pre += w[k] * ld(init, b * is_s0 + d * is_s1 + ii * is_s2, dtype);
                }
            }
            float o = apply_silu ? silu_f32(pre) : pre;            /* :108-111 */
            if (seq_idx && cur < 0) o = 0.0f;                     /* :113-115 */
            st(out, b * o_s0 + d * o_s1 + t * o_s2, dtype, o);    /* :117 */
        }
    }
    return 0;
}

/* ---- backward: bwd_full_cpu/kernel.mojo:25-314 -------------------------- */

typedef struct {
    int dtype, width, apply_silu;
    const void* x; int64_t xs0, xs1, xs2;
    const void* dout; int64_t gs0, gs1, gs2;
    const int32_t* seq; int64_t ss0, ss1;
    const void* init; int64_t is0, is1, is2;
    int64_t seqlen;
} bwd_ctx;

/* _cpu_dpre_at, bwd_full_cpu/kernel.mojo:25-105 */
static float dpre_at(const bwd_ctx* c, int64_t t, int64_t b, int64_t d,
                     float bias_v, const float* w) {
    const int64_t W = c->width;
    if (t < 0 || t >= c->seqlen) return 0.0f;                     /* :68-69 */
    int32_t cur = 0;
    if (c->seq) {
        cur = c->seq[b * c->ss0 + t * c->ss1];
        if (cur < 0) return 0.0f;                                  /* :75-77 */
    }
    const float g = ld(c->dout, b * c->gs0 + d * c->gs1 + t * c->gs2, c->dtype);
    if (!c->apply_silu) return g;                                  /* :79-80 */
    float pre = bias_v;
    for (int64_t k = 0; k < W; ++k) {                              /* :84-101 */
        const int64_t src = t + k - (W - 1);
        if (src >= 0) {
            int include = 1;
            if (c->seq) include = (c->seq[b * c->ss0 + src * c->ss1] == cur);
            if (include) pre += w[k] * ld(c->x, b * c->xs0 + d * c->xs1 + src * c->xs2, c->dtype);
        } else if (c->init) {
            const int64_t ii = src + (W - 1);
            pre += w[k] * ld(c->init, b * c->is0 + d * c->is1 + ii * c->is2, c->dtype);
        }
    }
    const float sig = 1.0f / (1.0f + expf(-pre));                  /* :102-105 */
    const float silu_grad = sig * (1.0f + pre * (1.0f - sig));
    return g * silu_grad;
}

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
               void* dinit, int64_t di_s0, int64_t di_s1, int64_t di_s2) {
    int rc = check_common(dtype, width);
    if (rc) return rc;
    if (!dweight_acc) return 3;
    if (init && !dinit) return 3;
    const int64_t W = width;
    const int64_t nbc = batch * dim;
    bwd_ctx c = {dtype, width, apply_silu, x, x_s0, x_s1, x_s2, dout, g_s0, g_s1, g_s2,
                 seq_idx, si_s0, si_s1, init, is_s0, is_s1, is_s2, seqlen};
    /* per-row partials, merged below in batch order */
    float* part_w = (float*)calloc((size_t)(nbc > 0 ? nbc : 1) * (size_t)W, sizeof(float));
    float* part_b = (float*)calloc((size_t)(nbc > 0 ? nbc : 1), sizeof(float));
    if (!part_w || !part_b) { free(part_w); free(part_b); return 4; }

#pragma omp parallel for schedule(static)
    for (int64_t bc = 0; bc < nbc; ++bc) {
        const int64_t b = bc / dim, d = bc % dim;
        float bias_v = 0.0f;
        if (bias) bias_v = ld(bias, d, dtype);                     /* :166-167 */
        float w[MAX_WIDTH];
        for (int64_t k = 0; k < W; ++k) w[k] = ld(weight, d * w_s0 + k * w_s1, dtype);
        float win[MAX_WIDTH];                                      /* dpre_win[k] = dpre[t+k] */
        for (int64_t k = 0; k < W; ++k) win[k] = dpre_at(&c, k, b, d, bias_v, w);
        float lw[MAX_WIDTH] = {0};
        float lb = 0.0f;
        if (init) {                                                /* :210-227 */
            for (int64_t i = 0; i < W - 1; ++i) {
                float v = 0.0f;
                for (int64_t k = 0; k < W; ++k)
                    if (i - k >= 0) v += w[k] * win[i - k];
                st(dinit, b * di_s0 + d * di_s1 + i * di_s2, dtype, v);
            }
            for (int64_t k = 0; k < W; ++k)
                for (int64_t t = 0; t < W - 1 - k; ++t)
                    lw[k] += win[t] * ld(init, b * is_s0 + d * is_s1 + (t + k) * is_s2, dtype);
        }
        for (int64_t t = 0; t < seqlen; ++t) {                     /* :229-300 */
            int32_t cur = 0;
            if (seq_idx) cur = seq_idx[b * si_s0 + t * si_s1];
            float dxv = 0.0f;
            for (int64_t k = 0; k < W; ++k) {                      /* :241-252 */
                int include = 1;
                if (seq_idx) {
                    const int64_t pk = t + k;
                    include = (pk < seqlen) ? (seq_idx[b * si_s0 + pk * si_s1] == cur) : 0;
                }
                if (include) dxv += w[W - 1 - k] * win[k];
            }
            st(dx, b * dx_s0 + d * dx_s1 + t * dx_s2, dtype, dxv);
            const float dp = win[0];
            if (bias) lb += dp;                                    /* :261-262 */
            for (int64_t k = 0; k < W; ++k) {                      /* :264-274 */
                const int64_t src = t + k - (W - 1);
                if (src >= 0) {
                    int include = 1;
                    if (seq_idx) include = (seq_idx[b * si_s0 + src * si_s1] == cur);
                    if (include) lw[k] += dp * ld(x, b * x_s0 + d * x_s1 + src * x_s2, dtype);
                }
            }
            for (int64_t k = 0; k < W - 1; ++k) win[k] = win[k + 1]; /* :277-300 */
            win[W - 1] = dpre_at(&c, t + W, b, d, bias_v, w);
        }
        for (int64_t k = 0; k < W; ++k) part_w[bc * W + k] = lw[k];
        part_b[bc] = lb;
    }
    /* :302-312 -- merge the per-(b, d) contributions */
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t d = 0; d < dim; ++d) {
            for (int64_t k = 0; k < W; ++k) dweight_acc[d * W + k] += part_w[(b * dim + d) * W + k];
            if (bias && dbias_acc) dbias_acc[d] += part_b[b * dim + d];
        }
    free(part_w);
    free(part_b);
    return 0;
}

/* ---- decode update: update_cpu/kernel.mojo:49-141 ----------------------- */

int oracle_update(int dtype, int width, int apply_silu,
                  const void* x, const void* weight, const void* bias,
                  void* conv_state, void* out,
                  int64_t batch, int64_t dim, int64_t seqlen, int64_t state_len,
                  int64_t x_s0, int64_t x_s1, int64_t x_s2,
                  int64_t w_s0, int64_t w_s1,
                  int64_t cs_s0, int64_t cs_s1, int64_t cs_s2,
                  int64_t o_s0, int64_t o_s1, int64_t o_s2,
                  const int32_t* state_indices, const int32_t* cache_seqlens) {
    int rc = check_common(dtype, width);
    if (rc) return rc;
    const int64_t W = width;
    if (state_len < W - 1) return 5;
    const int64_t nbc = batch * dim;
#pragma omp parallel for schedule(static)
    for (int64_t bc = 0; bc < nbc; ++bc) {
        const int64_t b = bc / dim, d = bc % dim;
        int64_t row = b;
        if (state_indices) {                                       /* :58-64 */
            const int64_t iv = state_indices[b];
            if (iv < 0) {
                for (int64_t i = 0; i < seqlen; ++i) st(out, b * o_s0 + d * o_s1 + i * o_s2, dtype, 0.0f);
                continue;
            }
            row = iv;
        }
        float w[MAX_WIDTH];
        for (int64_t k = 0; k < W; ++k) w[k] = ld(weight, d * w_s0 + k * w_s1, dtype);
        float bias_v = 0.0f;
        if (bias) bias_v = ld(bias, d, dtype);
        const int64_t sbase = row * cs_s0 + d * cs_s1;
        int64_t upd = 0;
        if (cache_seqlens) {                                       /* :78-82 */
            int64_t cs = (int64_t)cache_seqlens[b] % state_len;
            if (cs < 0) cs += state_len; /* floored modulo, as torch.remainder */
            upd = cs - (W - 1);
            if (upd < 0) upd += state_len;
        }
        const int64_t adv = seqlen;
        float xv[MAX_WIDTH] = {0};
        if (!cache_seqlens) {
            for (int64_t i = 0; i < state_len - adv - (W - 1); ++i)  /* :89-92 */
                st(conv_state, sbase + i * cs_s2, dtype, ld(conv_state, sbase + (i + adv) * cs_s2, dtype));
            for (int64_t i = 0; i < W - 1; ++i) {                    /* :96-102 */
                const int64_t ridx = state_len - (W - 1) + i;
                const float sv = ld(conv_state, sbase + ridx * cs_s2, dtype);
                const int64_t widx = state_len - adv - (W - 1) + i;
                if (i < adv + (W - 1) && widx >= 0) st(conv_state, sbase + widx * cs_s2, dtype, sv);
                xv[i] = sv;
            }
        } else {
            for (int64_t i = 0; i < W - 1; ++i) {                    /* :105-110 */
                xv[i] = ld(conv_state, sbase + upd * cs_s2, dtype);
                if (++upd >= state_len) upd -= state_len;
            }
        }
        for (int64_t i = 0; i < seqlen; ++i) {                     /* :113-139 */
            const float xi = ld(x, b * x_s0 + d * x_s1 + i * x_s2, dtype);
            if (!cache_seqlens) {
                const int64_t widx = state_len - adv + i;
                if (i < adv && widx >= 0) st(conv_state, sbase + widx * cs_s2, dtype, xi);
            } else {
                st(conv_state, sbase + upd * cs_s2, dtype, xi);
                if (++upd >= state_len) upd -= state_len;
            }
            xv[W - 1] = xi;
            float o = bias_v;
            for (int64_t k = 0; k < W; ++k) o += w[k] * xv[k];
            if (apply_silu) o = silu_f32(o);
            st(out, b * o_s0 + d * o_s1 + i * o_s2, dtype, o);
            for (int64_t k = 0; k < W - 1; ++k) xv[k] = xv[k + 1];
        }
    }
    return 0;
}
