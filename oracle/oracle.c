/*
 * oracle.c -- CPU restatement of the reference's quantized-matmul and MoE path.
 *
 * TEST INFRASTRUCTURE ONLY: what the HIP kernels are compared against, and the "port" CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Build with -ffp-contract=off and without fast-math: every float operation below is one IEEE
 * F32 operation, as in the Rust reference (which never contracts) and in ggml built with the
 * reference's flags (crates/kernels-ggml/build.rs:187-210).
 *
 * Pins (what checks each part; the tests under tests/ run them):
 *   conversions      every F16 pattern round trip; f16_bits against IEEE RNE (numpy float16)
 *                    and the ggml-q8.txt f16/bf16 lines
 *   or_exp/or_silu   within 2 ulp of F64 exp on a bit-pattern sweep; the edge cases of
 *                    crates/kernels/src/reference/math/tests.rs
 *   or_sum/or_dot    brute-force level-by-level tree (reduce.rs module docs), small cases
 *   or_quantize      FNV-1a digests of crates/kernels-ggml/tests/quantize.rs:114-138, and
 *                    ggml's own quantizers compiled into oracle/_ref where the reference is
 *                    present
 *   act quantizers   crates/kernels/tests/data/act_quant/ggml-q8.txt (q8_0 cpu = Arm64Neon,
 *                    q8_0/q8_1 ref, q8_K)
 *   or_gemv          pinned output bits of crates/kernels-cpu/src/gemv/tests.rs:739-777 and
 *                    the hand-computed cases at :407-458, plus the F64 derived bound
 *   or_gate_up_act   or_gemv and or_silu composed; a one-hot Q8_0 gate/up pair pins the row
 *                    order (gate rows first) and the product against the activation codes
 *   or_rms_norm      the edge cases of norm.rs's docs (zeros, eps 0, NaN, infinity), a hand
 *                    case whose bits follow from the operation order, and an F64 bound
 *   or_logits        or_rms_norm and or_gemv composed; rows whose norm is an exact halving pin
 *                    that the norm comes first and that g scales its own column
 *   or_moe_*         packing against brute force; MoE slot = expert FFN of the row alone
 *                    (moe/tests.rs:315); combine against its definition; the rank-order
 *                    combine equal to it on rows whose ids ascend, and on order-sensitive hand
 *                    cases; route ids against a brute-force sort.  MoeRoute and MoeCombine have no reference code: their
 *                    values are pinned by the specification and invariants only.
 *   or_moe_assign    the reference's generated split rule (moe_assign.h), compiled into
 *                    oracle/_ref, on 10^6 generated inputs; the hand-worked cases of
 *                    crates/kernels/src/moe/tests.rs:801-922
 *   or_moe_doorbell  struct layout against moe_doorbell.h compiled into oracle/_ref; the
 *                    byte example of moe/tests.rs:938-961; the route list against a brute-force
 *                    count of the ids
 */
/* The weight quantizers restate ggml (Copyright (c) 2023-2026 The ggml authors, MIT License;
 * the notice is in THIRD_PARTY.md at the repository root). */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define QK32 32
#define QK_K 256

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline int is_finite_f(float v) { return (f2u(v) & 0x7F800000u) != 0x7F800000u; }

/* ===================================================================================== */
/* Conversions: crates/kernels/src/reference/act_quant.rs:398-485                         */
/* ===================================================================================== */

/* act_quant.rs:400-446 f16_bits: round to nearest even, subnormals kept, NaN -> sign|0x7E00 */
uint16_t or_f16_bits(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t abs_ = b & 0x7FFFFFFFu;
    if (abs_ > 0x7F800000u) return sign | 0x7E00u;
    if (abs_ >= 0x477FF000u) return sign | 0x7C00u;
    int exp = (int)(abs_ >> 23) - 127;
    uint32_t mant = abs_ & 0x007FFFFFu;
    uint64_t base, rem, half;
    if (exp >= -14) {
        base = ((uint64_t)(exp + 15) << 10) | (mant >> 13);
        rem = mant & 0x1FFFu;
        half = 0x1000u;
    } else if (abs_ < 0x00800000u) {
        base = 0;
        rem = 0;
        half = 1;
    } else {
        uint64_t sig = (uint64_t)(mant | 0x00800000u);
        uint32_t shift = (uint32_t)(-exp - 1);
        if (shift >= 40) {
            base = 0;
            rem = 0;
            half = 1;
        } else {
            base = sig >> shift;
            uint64_t r = sig & ((1ull << shift) - 1);
            uint64_t h = 1ull << (shift - 1);
            rem = r < h ? 0 : (r == h ? 1 : 2);
            half = 1;
        }
    }
    uint64_t rounded = (rem > half || (rem == half && (base & 1))) ? base + 1 : base;
    return (uint16_t)(sign | (uint16_t)rounded);
}

/* act_quant.rs:448-467 f16_to_f32: exact */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x03FFu;
    uint32_t bits;
    if (exp == 0 && mant == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t lead = 31 - (uint32_t)__builtin_clz(mant);
        uint32_t e = lead + 127 - 24;
        bits = sign | (e << 23) | ((mant << (23 - lead)) & 0x007FFFFFu);
    } else if (exp == 0x1F && mant == 0) {
        bits = sign | 0x7F800000u;
    } else if (exp == 0x1F) {
        bits = sign | 0x7FC00000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return u2f(bits);
}

/* act_quant.rs:472-479 round_bf16 */
uint16_t or_round_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 64u);
    return (uint16_t)(((uint64_t)u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* act_quant.rs:481-485 */
float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* ===================================================================================== */
/* Software exp / silu: crates/kernels/src/reference/math.rs:15-84                        */
/* ===================================================================================== */

static inline float pow2_f(int k) { return u2f((uint32_t)(k + 127) << 23); }

float or_exp(float x) {
    const float LOG2_E = 1.44269504088896340736f;
    const float LN2_HI = u2f(0x3F317200u);
    const float LN2_LO = 1.4286068e-6f;
    const float OVERFLOW_ = 88.72284f;
    const float UNDERFLOW_ = -103.97208f;
    if (x != x) return x + x;
    if (x > OVERFLOW_) return INFINITY;
    if (x < UNDERFLOW_) return 0.0f;
    float kf = nearbyintf(x * LOG2_E);
    float r = (x - kf * LN2_HI) - kf * LN2_LO;
    const float C[8] = {1.0f,         1.0f,          0.5f,          1.0f / 6.0f,
                        1.0f / 24.0f, 1.0f / 120.0f, 1.0f / 720.0f, 1.0f / 5040.0f};
    float p = C[7];
    for (int i = 6; i >= 0; --i) p = p * r + C[i];
    int k = (int)kf;
    /* Rust div_euclid(2): floor division for a positive divisor */
    int k1 = (k >= 0) ? k / 2 : -((-k + 1) / 2);
    return (p * pow2_f(k1)) * pow2_f(k - k1);
}

float or_silu(float x) { return x / (1.0f + or_exp(-x)); }

/* The worst distance of or_exp from F64 exp, in units of the F32 spacing at the true value,
 * over every `step`-th bit pattern of each sign in exp's finite range: the check of
 * crates/kernels/src/reference/math/tests.rs:19-40, which bounds it by 2. */
double or_exp_worst_ulp(uint32_t step) {
    double worst = 0.0;
    for (uint64_t bits = 0; bits < 0x80000000ull; bits += step) {
        for (int sgn = 0; sgn < 2; ++sgn) {
            float x = u2f((uint32_t)bits | (sgn ? 0x80000000u : 0u));
            if (!(x >= -103.97208f && x <= 88.72283f)) continue;
            double want = exp((double)x);
            double spacing = fabs(want) < 1.1754943508222875e-38 ? ldexp(1.0, -149)
                                                                 : ldexp(1.0, (int)floor(log2(fabs(want))) - 23);
            double err = fabs((double)or_exp(x) - want) / spacing;
            if (err > worst) worst = err;
        }
    }
    return worst;
}

/* ===================================================================================== */
/* F32Fixed reductions: crates/kernels/src/reference/reduce.rs:30-90                      */
/* ===================================================================================== */

static float sum_terms(size_t n, const float* a, const float* b) {
    float sums[64];
    uint32_t levels[64];
    size_t depth = 0, start = 0;
    while (start < n) {
        size_t end = n < start + 32 ? n : start + 32;
        float acc = 0.0f;
        for (size_t i = start; i < end; ++i) acc += b ? a[i] * b[i] : a[i];
        uint32_t level = 0;
        while (depth > 0 && levels[depth - 1] == level) {
            depth -= 1;
            acc = sums[depth] + acc;
            level += 1;
        }
        sums[depth] = acc;
        levels[depth] = level;
        depth += 1;
        start = end;
    }
    if (depth == 0) return 0.0f;
    float acc = sums[depth - 1];
    for (size_t i = depth - 1; i-- > 0;) acc = sums[i] + acc;
    return acc;
}

float or_sum(const float* xs, size_t n) { return sum_terms(n, xs, NULL); }
float or_dot(const float* a, const float* b, size_t n) { return sum_terms(n, a, b); }

/* ===================================================================================== */
/* Geometry: crates/kernels/src/reference/dequant.rs:46-84, kernels-cpu/src/gemv.rs:119-151 */
/* ===================================================================================== */

int or_block_elems(int ty) {
    switch (ty) {
    case OR_F16:
    case OR_BF16: return 1;
    case OR_Q8_0:
    case OR_Q4_0: return QK32;
    case OR_Q4_K: return QK_K;
    default: return 0;
    }
}

int or_block_bytes(int ty) {
    switch (ty) {
    case OR_F16:
    case OR_BF16: return 2;
    case OR_Q8_0: return 34;
    case OR_Q4_0: return 18;
    case OR_Q4_K: return 144;
    default: return 0;
    }
}

int or_act_kind(int ty) {
    switch (ty) {
    case OR_Q8_0:
    case OR_Q4_0: return OR_ACT_Q8_0;
    case OR_Q4_K: return OR_ACT_Q8K;
    default: return OR_ACT_F32;
    }
}

/* ===================================================================================== */
/* Exact dequant: crates/kernels/src/reference/dequant.rs:116-173                         */
/* ===================================================================================== */

static inline float half_at(const uint8_t* b) { return or_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* dequant.rs:122-131 / gemv.rs:528-537 get_scale_min_k4 */
static inline void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

int or_dequantize(int ty, const uint8_t* src, size_t nbytes, float* out) {
    int bb = or_block_bytes(ty), be = or_block_elems(ty);
    if (!bb || nbytes % (size_t)bb) return -1;
    size_t nb = nbytes / (size_t)bb;
    for (size_t i = 0; i < nb; ++i) {
        const uint8_t* blk = src + i * (size_t)bb;
        float* y = out + i * (size_t)be;
        switch (ty) {
        case OR_F16: y[0] = half_at(blk); break;
        case OR_BF16: y[0] = or_bf16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))); break;
        case OR_Q8_0: {
            float d = half_at(blk);
            for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)blk[2 + j] * d;
            break;
        }
        case OR_Q4_0: {
            float d = half_at(blk);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)((int)(blk[2 + j] & 0x0F) - 8) * d;
                y[j + 16] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
            }
            break;
        }
        case OR_Q4_K: {
            float d = half_at(blk), mn = half_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qs = blk + 16;
            for (int g = 0; g < 4; ++g) {
                uint8_t sc, m;
                scale_min_k4(2 * g, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = mn * (float)m;
                scale_min_k4(2 * g + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = mn * (float)m;
                for (int l = 0; l < 32; ++l) {
                    y[64 * g + l] = d1 * (float)(qs[32 * g + l] & 0xF) - m1;
                    y[64 * g + 32 + l] = d2 * (float)(qs[32 * g + l] >> 4) - m2;
                }
            }
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

/* ===================================================================================== */
/* Weight quantizers: third_party/ggml/src/ggml-quants.c                                   */
/* ===================================================================================== */

/* ggml-quants.c:621-626 nearest_int (also kernels-cpu/src/gemv/act.rs:345-348) */
static inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* ggml-quants.c:113-140 quantize_row_q4_0_ref */
static void quantize_q4_0(const float* x, uint8_t* y, size_t k) {
    size_t nb = k / 32;
    for (size_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        uint16_t dh = or_f16_bits(d);
        uint8_t* blk = y + i * 18;
        blk[0] = (uint8_t)dh;
        blk[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[i * 32 + j] * id;
            const float x1 = x[i * 32 + 16 + j] * id;
            int8_t t0 = (int8_t)(x0 + 8.5f);
            int8_t t1 = (int8_t)(x1 + 8.5f);
            const uint8_t xi0 = (uint8_t)(t0 < 15 ? t0 : 15);
            const uint8_t xi1 = (uint8_t)(t1 < 15 ? t1 : 15);
            blk[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

/* ggml-quants.c:276-297 quantize_row_q8_0_ref */
static void quantize_q8_0(const float* x, uint8_t* y, size_t k) {
    size_t nb = k / 32;
    for (size_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            float a = fabsf(v);
            amax = amax > a ? amax : a; /* ggml's MAX(amax, fabsf(v)) */
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        uint16_t dh = or_f16_bits(d);
        uint8_t* blk = y + i * 34;
        blk[0] = (uint8_t)dh;
        blk[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 32; ++j) {
            const float x0 = x[i * 32 + j] * id;
            blk[2 + j] = (uint8_t)(int8_t)roundf(x0);
        }
    }
}

/* ggml-quants.c:799-878 make_qkx2_quants (use_mad = false on every call site here) */
static float make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L,
                              float* the_min, uint8_t* Laux, float rmin, float rdelta,
                              int nstep) {
    float min = x[0];
    float max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        l = l < nmax ? l : nmax;
        L[i] = (uint8_t)(l > 0 ? l : 0);
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        float w = weights[i];
        best_error += w * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < nmax ? l : nmax;
            l = l > 0 ? l : 0;
            Laux[i] = (uint8_t)l;
            float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                float w = weights[i];
                cur_error += w * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* ggml-quants.c:1458-1528 quantize_row_q4_K_ref */
static void quantize_q4_k(const float* x, uint8_t* y, size_t k) {
    size_t nb = k / QK_K;
    uint8_t L[QK_K];
    uint8_t Laux[32];
    float weights[32];
    float mins[QK_K / 32];
    float scales[QK_K / 32];
    for (size_t i = 0; i < nb; i++) {
        uint8_t* blk = y + i * 144;
        uint8_t* bsc = blk + 4;
        memset(bsc, 0, 12);
        float max_scale = 0;
        float max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux,
                                         -1.f, 0.1f, 20);
            float scale = scales[j];
            if (scale > max_scale) max_scale = scale;
            float min = mins[j];
            if (min > max_min) max_min = min;
        }
        float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                bsc[j] = ls;
                bsc[j + 4] = lm;
            } else {
                bsc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                bsc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                bsc[j - 0] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        uint16_t dh = or_f16_bits(max_scale / 63.f);
        uint16_t mh = or_f16_bits(max_min / 63.f);
        blk[0] = (uint8_t)dh;
        blk[1] = (uint8_t)(dh >> 8);
        blk[2] = (uint8_t)mh;
        blk[3] = (uint8_t)(mh >> 8);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            scale_min_k4(j, bsc, &sc, &m);
            const float d = or_f16_to_f32(dh) * sc;
            if (!d) continue;
            const float dm = or_f16_to_f32(mh) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 15 ? l : 15;
                l = l > 0 ? l : 0;
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t* q = blk + 16;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

long or_quantize(int ty, const float* x, size_t n, uint8_t* out) {
    int be = or_block_elems(ty);
    if (!be || n % (size_t)be) return -1;
    switch (ty) {
    case OR_Q4_0: quantize_q4_0(x, out, n); break;
    case OR_Q8_0: quantize_q8_0(x, out, n); break;
    case OR_Q4_K: quantize_q4_k(x, out, n); break;
    case OR_F16:
        for (size_t i = 0; i < n; ++i) {
            uint16_t h = or_f16_bits(x[i]);
            out[2 * i] = (uint8_t)h;
            out[2 * i + 1] = (uint8_t)(h >> 8);
        }
        break;
    case OR_BF16:
        for (size_t i = 0; i < n; ++i) {
            uint16_t h = or_round_bf16(x[i]);
            out[2 * i] = (uint8_t)h;
            out[2 * i + 1] = (uint8_t)(h >> 8);
        }
        break;
    default: return -1;
    }
    return (long)(n / (size_t)be * (size_t)or_block_bytes(ty));
}

/* ===================================================================================== */
/* Reference activation quantizers in ggml byte layouts:                                  */
/* crates/kernels/src/reference/act_quant.rs:241-393                                      */
/* ===================================================================================== */

/* act_quant.rs:250-281 q8_block; returns 0 for a non-finite block */
static int q8_block_ref(const float* x, int path, float* d_out, int8_t* qs) {
    for (int i = 0; i < 32; ++i)
        if (!is_finite_f(x[i])) return 0;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float a = fabsf(x[i]);
        amax = amax > a ? amax : a;
    }
    float d = amax / 127.0f;
    float id;
    if ((path == 0 || path == 1) && d != 0.0f) id = 1.0f / d;
    else if (path == 2 && amax != 0.0f) id = 127.0f / amax;
    else id = 0.0f;
    memset(qs, 0, 32);
    if (is_finite_f(id)) {
        for (int i = 0; i < 32; ++i) {
            float t = x[i] * id;
            float r = path == 0 ? roundf(t) : nearbyintf(t);
            qs[i] = (int8_t)(int)r;
        }
    }
    *d_out = d;
    return 1;
}

int or_quantize_q8_0_blocks(const float* x, size_t n, int path, uint8_t* out) {
    if (n % 32) return -1;
    for (size_t b = 0; b < n / 32; ++b) {
        uint8_t* o = out + b * 34;
        float d;
        int8_t qs[32];
        uint16_t dh;
        if (q8_block_ref(x + b * 32, path, &d, qs)) {
            dh = or_f16_bits(d);
        } else {
            dh = 0x7E00;
            memset(qs, 0, 32);
        }
        o[0] = (uint8_t)dh;
        o[1] = (uint8_t)(dh >> 8);
        memcpy(o + 2, qs, 32);
    }
    return 0;
}

int or_quantize_q8_1_blocks(const float* x, size_t n, int path, uint8_t* out) {
    if (n % 32) return -1;
    for (size_t b = 0; b < n / 32; ++b) {
        uint8_t* o = out + b * 36;
        float d;
        int8_t qs[32];
        uint16_t dh, sh;
        if (q8_block_ref(x + b * 32, path, &d, qs)) {
            int sum = 0;
            for (int i = 0; i < 32; ++i) sum += qs[i];
            float s = (float)sum * d;
            dh = or_f16_bits(d);
            sh = or_f16_bits(s);
        } else {
            dh = 0x7E00;
            sh = 0x7E00;
            memset(qs, 0, 32);
        }
        o[0] = (uint8_t)dh;
        o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)sh;
        o[3] = (uint8_t)(sh >> 8);
        memcpy(o + 4, qs, 32);
    }
    return 0;
}

/* act_quant.rs:343-380 q8_k_block, in ggml's block_q8_K layout (d, qs[256], bsums[16]) */
int or_quantize_q8_k_blocks(const float* x, size_t n, uint8_t* out) {
    if (n % QK_K) return -1;
    for (size_t b = 0; b < n / QK_K; ++b) {
        const float* xb = x + b * QK_K;
        uint8_t* o = out + b * 292;
        float d = 0.0f;
        int8_t qs[QK_K];
        int16_t bsums[16];
        memset(qs, 0, sizeof qs);
        memset(bsums, 0, sizeof bsums);
        int finite = 1;
        for (int i = 0; i < QK_K; ++i)
            if (!is_finite_f(xb[i])) finite = 0;
        if (!finite) {
            d = NAN;
        } else {
            float amax = 0.0f, max = 0.0f;
            for (int i = 0; i < QK_K; ++i)
                if (fabsf(xb[i]) > amax) {
                    amax = fabsf(xb[i]);
                    max = xb[i];
                }
            if (amax != 0.0f) {
                float iscale = -127.0f / max;
                if (is_finite_f(iscale)) {
                    for (int i = 0; i < QK_K; ++i) {
                        int q = nearest_int(iscale * xb[i]);
                        qs[i] = (int8_t)(q < 127 ? q : 127);
                    }
                    for (int j = 0; j < 16; ++j) {
                        int s = 0;
                        for (int i = 0; i < 16; ++i) s += qs[16 * j + i];
                        bsums[j] = (int16_t)s;
                    }
                }
                d = 1.0f / iscale;
            }
        }
        memcpy(o, &d, 4);
        memcpy(o + 4, qs, QK_K);
        memcpy(o + 4 + QK_K, bsums, 32);
    }
    return 0;
}

/* ===================================================================================== */
/* GEMV activations: crates/kernels-cpu/src/gemv/act.rs                                    */
/* ===================================================================================== */

static void act_counts(int kind, size_t n, size_t* codes, size_t* scales, size_t* sums) {
    switch (kind) {
    case OR_ACT_Q8_0: *codes = n; *scales = n / QK32; *sums = 0; break;
    case OR_ACT_Q8K: *codes = n; *scales = n / QK_K; *sums = n / QK32; break;
    default: *codes = *scales = *sums = 0;
    }
}

/* act.rs:108-111 */
size_t or_act_workspace_bytes(int kind, size_t rows, size_t k) {
    size_t c, s, m;
    act_counts(kind, rows * k, &c, &s, &m);
    return 4 * (s + m) + c;
}

/* act.rs:323-342 q8_0_block: ggml's arm64 quantizer; returns the scale the product uses */
static float q8_0_act_block(const float* x, int8_t* qs) {
    for (int i = 0; i < 32; ++i)
        if (!is_finite_f(x[i])) {
            memset(qs, 0, 32);
            return NAN;
        }
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float a = fabsf(x[i]);
        amax = amax > a ? amax : a;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    if (is_finite_f(id)) {
        for (int i = 0; i < 32; ++i) qs[i] = (int8_t)(int)nearbyintf(x[i] * id);
    } else {
        memset(qs, 0, 32);
    }
    return or_f16_to_f32(or_f16_bits(d));
}

/* act.rs:351-373 q8_k_block */
static float q8_k_act_block(const float* x, int8_t* qs) {
    memset(qs, 0, QK_K);
    for (int i = 0; i < QK_K; ++i)
        if (!is_finite_f(x[i])) return NAN;
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < QK_K; ++i)
        if (fabsf(x[i]) > amax) {
            amax = fabsf(x[i]);
            max = x[i];
        }
    if (amax == 0.0f) return 0.0f;
    float iscale = -127.0f / max;
    if (is_finite_f(iscale)) {
        for (int i = 0; i < QK_K; ++i) {
            int q = nearest_int(iscale * x[i]);
            qs[i] = (int8_t)(q < 127 ? q : 127);
        }
    }
    return 1.0f / iscale;
}

/* act.rs:71-101 fill, into the workspace layout of act.rs:122-167 */
int or_act_quantize(int kind, const float* x, size_t rows, size_t k, uint8_t* ws) {
    size_t n = rows * k, c, s, m;
    act_counts(kind, n, &c, &s, &m);
    if (kind == OR_ACT_F32) return 0;
    size_t blk = kind == OR_ACT_Q8_0 ? QK32 : QK_K;
    if (k % blk) return -1;
    float* d = (float*)ws;
    int32_t* sums = (int32_t*)(ws + 4 * s);
    int8_t* qs = (int8_t*)(ws + 4 * (s + m));
    for (size_t b = 0; b < n / blk; ++b) {
        d[b] = kind == OR_ACT_Q8_0 ? q8_0_act_block(x + b * blk, qs + b * blk)
                                   : q8_k_act_block(x + b * blk, qs + b * blk);
    }
    if (kind == OR_ACT_Q8K) {
        for (size_t j = 0; j < m; ++j) {
            int32_t t = 0;
            for (int i = 0; i < 32; ++i) t += qs[j * 32 + i];
            sums[j] = t;
        }
    }
    return 0;
}

/* ===================================================================================== */
/* GEMV: crates/kernels-cpu/src/gemv.rs, gemv/portable.rs                                  */
/* ===================================================================================== */

/* gemv.rs:539-547 */
static inline float q4k_term(float d, float dmin, float dx, int32_t s1, int32_t s2) {
    return (d * dx) * (float)s1 - (dmin * dx) * (float)s2;
}
static inline float q32_term(float dw, float dx, int32_t s) { return (dw * dx) * (float)s; }

/* portable.rs:30-45 float_rows with the lane fold of gemv.rs:506-516 */
static void float_rows(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x,
                       size_t rows, size_t o0, size_t o1, float* y) {
    for (size_t o = o0; o < o1; ++o) {
        const uint8_t* wr = w + o * k * 2;
        for (size_t r = 0; r < rows; ++r) {
            const float* xr = x + r * k;
            float lanes[32];
            for (int l = 0; l < 32; ++l) lanes[l] = 0.0f;
            for (size_t i = 0; i < k; ++i) {
                uint16_t h = (uint16_t)(wr[2 * i] | (wr[2 * i + 1] << 8));
                float wv = ty == OR_F16 ? or_f16_to_f32(h) : or_bf16_to_f32(h);
                lanes[i % 32] = fmaf(wv, xr[i], lanes[i % 32]);
            }
            for (int h = 16; h > 0; h /= 2)
                for (int j = 0; j < h; ++j) lanes[j] += lanes[j + h];
            y[r * n_out + o] = lanes[0];
        }
    }
}

/* portable.rs:114-190 int_rows: exact i32 block sums, one F32 term per block, added in block
 * order from +0.0.  Row groups (ROW_GROUP = 8) only change how often a block is re-read, not
 * any value, so each activation row is folded on its own here. */
static void int_rows(int ty, const uint8_t* w, size_t n_out, size_t k, const uint8_t* ws,
                     size_t rows, size_t o0, size_t o1, float* y) {
    int kind = or_act_kind(ty);
    size_t n = rows * k, c, s, m;
    act_counts(kind, n, &c, &s, &m);
    const float* xd = (const float*)ws;
    const int32_t* xs = (const int32_t*)(ws + 4 * s);
    const int8_t* xq = (const int8_t*)(ws + 4 * (s + m));
    size_t be = (size_t)or_block_elems(ty), bb = (size_t)or_block_bytes(ty);
    size_t nb = k / be, row_bytes = nb * bb;
    for (size_t r = 0; r < rows; ++r) {
        const int8_t* qx = xq + r * k;
        const float* dx = xd + r * (k / be);
        const int32_t* sx = kind == OR_ACT_Q8K ? xs + r * (k / 32) : NULL;
        for (size_t o = o0; o < o1; ++o) {
            const uint8_t* wr = w + o * row_bytes;
            float acc = 0.0f;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = wr + b * bb;
                const int8_t* xb = qx + b * be;
                if (ty == OR_Q8_0) {
                    int32_t sum = 0;
                    for (int i = 0; i < 32; ++i) sum += (int32_t)(int8_t)blk[2 + i] * xb[i];
                    acc += q32_term(half_at(blk), dx[b], sum);
                } else if (ty == OR_Q4_0) {
                    int32_t sum = 0;
                    for (int i = 0; i < 16; ++i) {
                        uint8_t q = blk[2 + i];
                        sum += ((int32_t)(q & 0xF) - 8) * xb[i] + ((int32_t)(q >> 4) - 8) * xb[16 + i];
                    }
                    acc += q32_term(half_at(blk), dx[b], sum);
                } else { /* Q4_K */
                    int32_t sb[8];
                    const uint8_t* q = blk + 16;
                    for (int g = 0; g < 4; ++g) {
                        int32_t lo = 0, hi = 0;
                        for (int l = 0; l < 32; ++l) {
                            lo += (int32_t)(q[32 * g + l] & 0xF) * xb[64 * g + l];
                            hi += (int32_t)(q[32 * g + l] >> 4) * xb[64 * g + 32 + l];
                        }
                        sb[2 * g] = lo;
                        sb[2 * g + 1] = hi;
                    }
                    int32_t s1 = 0, s2 = 0;
                    for (int j = 0; j < 8; ++j) {
                        uint8_t sc, mn;
                        scale_min_k4(j, blk + 4, &sc, &mn);
                        s1 += (int32_t)sc * sb[j];
                        s2 += (int32_t)mn * sx[b * 8 + j];
                    }
                    acc += q4k_term(half_at(blk), half_at(blk + 2), dx[b], s1, s2);
                }
            }
            y[r * n_out + o] = acc;
        }
    }
}

/* ===================================================================================== */
/* The reference's x86 level of the same kernel (crates/kernels-cpu/src/gemv/x86.rs:74-153;  */
/* portable.rs:114-190 int_rows with gemv.rs:83 ROW_GROUP = 8): a block's weights are loaded */
/* once for up to 8 activation rows, and each exact block sum comes from AVX2 byte products: */
/* |w| as unsigned bytes times x * sign(w) as signed bytes (vpmaddubsw cannot saturate:       */
/* |w| <= 128, |x| <= 127), pairs summed by vpmaddwd, then a horizontal add.  The sums are     */
/* exact, the F32 terms and their order are int_rows', so the outputs are its bits (the tests */
/* compare them).  This is the timed CPU baseline; the portable form above is the reference  */
/* restatement the tests compare the GPU outputs with.                                        */
/* ===================================================================================== */
#include <immintrin.h>

#define OR_ROW_GROUP 8

static inline int32_t x86_hsum(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}
/* sum over 32 signed byte pairs, exact */
static inline int32_t x86_dot_i8(__m256i w, __m256i x) {
    const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(x, w));
    return x86_hsum(_mm256_madd_epi16(p, _mm256_set1_epi16(1)));
}
/* sum over 32 pairs of unsigned bytes n <= 15 and signed bytes x, exact */
static inline int32_t x86_dot_u4(__m256i n, __m256i x) {
    return x86_hsum(_mm256_madd_epi16(_mm256_maddubs_epi16(n, x), _mm256_set1_epi16(1)));
}
static inline __m256i x86_load32(const void* p) { return _mm256_loadu_si256((const __m256i*)p); }

static void int_rows_x86(int ty, const uint8_t* w, size_t n_out, size_t k, const uint8_t* ws,
                         size_t rows, size_t o0, size_t o1, float* y) {
    int kind = or_act_kind(ty);
    size_t n = rows * k, c, s, m;
    act_counts(kind, n, &c, &s, &m);
    const float* xd = (const float*)ws;
    const int32_t* xs = (const int32_t*)(ws + 4 * s);
    const int8_t* xq = (const int8_t*)(ws + 4 * (s + m));
    size_t be = (size_t)or_block_elems(ty), bb = (size_t)or_block_bytes(ty);
    size_t nb = k / be, row_bytes = nb * bb;
    const __m256i low4 = _mm256_set1_epi8(0x0F);
    for (size_t r0 = 0; r0 < rows; r0 += OR_ROW_GROUP) {
        const size_t nr = rows - r0 < OR_ROW_GROUP ? rows - r0 : OR_ROW_GROUP;
        for (size_t o = o0; o < o1; ++o) {
            const uint8_t* wr = w + o * row_bytes;
            float acc[OR_ROW_GROUP];
            for (size_t i = 0; i < nr; ++i) acc[i] = 0.0f;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t* blk = wr + b * bb;
                if (ty == OR_Q8_0 || ty == OR_Q4_0) {
                    __m256i wv;
                    if (ty == OR_Q8_0) {
                        wv = x86_load32(blk + 2);
                    } else { /* the 16 code bytes: low nibbles are values 0-15, high 16-31, minus 8 */
                        const __m128i q = _mm_loadu_si128((const __m128i*)(blk + 2));
                        const __m128i m4 = _mm_set1_epi8(0x0F);
                        wv = _mm256_sub_epi8(_mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(q, 4), m4),
                                                              _mm_and_si128(q, m4)),
                                             _mm256_set1_epi8(8));
                    }
                    const float dw = half_at(blk);
                    for (size_t i = 0; i < nr; ++i) {
                        const int32_t sum = x86_dot_i8(wv, x86_load32(xq + (r0 + i) * k + b * 32));
                        acc[i] += q32_term(dw, xd[(r0 + i) * nb + b], sum);
                    }
                } else { /* Q4_K: four groups of 64 values, low nibbles sub-block 2g, high 2g + 1 */
                    int32_t sb[OR_ROW_GROUP][8];
                    for (int g = 0; g < 4; ++g) {
                        const __m256i q = x86_load32(blk + 16 + 32 * g);
                        const __m256i lo = _mm256_and_si256(q, low4);
                        const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), low4);
                        for (size_t i = 0; i < nr; ++i) {
                            const int8_t* xb = xq + (r0 + i) * k + b * 256 + 64 * g;
                            sb[i][2 * g] = x86_dot_u4(lo, x86_load32(xb));
                            sb[i][2 * g + 1] = x86_dot_u4(hi, x86_load32(xb + 32));
                        }
                    }
                    int32_t sc[8], mn[8];
                    for (int j = 0; j < 8; ++j) {
                        uint8_t a, mm;
                        scale_min_k4(j, blk + 4, &a, &mm);
                        sc[j] = a;
                        mn[j] = mm;
                    }
                    const float d = half_at(blk), dmin = half_at(blk + 2);
                    for (size_t i = 0; i < nr; ++i) {
                        const int32_t* sx = xs + (r0 + i) * (k / 32) + b * 8;
                        int32_t s1 = 0, s2 = 0;
                        for (int j = 0; j < 8; ++j) {
                            s1 += sc[j] * sb[i][j];
                            s2 += mn[j] * sx[j];
                        }
                        acc[i] += q4k_term(d, dmin, xd[(r0 + i) * nb + b], s1, s2);
                    }
                }
            }
            for (size_t i = 0; i < nr; ++i) y[(r0 + i) * n_out + o] = acc[i];
        }
    }
}

/* level 0: the portable kernels; 1: the x86 level (integer types; the float types have one form) */
static int gemv_ws_level(int level, int ty, const uint8_t* w, size_t n_out, size_t k, const uint8_t* ws,
                         const float* xf, size_t rows, size_t o0, size_t o1, float* y) {
    if (!or_block_elems(ty) || k % (size_t)or_block_elems(ty) || o1 > n_out) return -1;
    if (rows == 0 || o0 >= o1) return 0;
    if (ty == OR_F16 || ty == OR_BF16) float_rows(ty, w, n_out, k, xf, rows, o0, o1, y);
    else if (level == 1) int_rows_x86(ty, w, n_out, k, ws, rows, o0, o1, y);
    else int_rows(ty, w, n_out, k, ws, rows, o0, o1, y);
    return 0;
}

int or_gemv_ws(int ty, const uint8_t* w, size_t n_out, size_t k, const uint8_t* ws,
               const float* xf, size_t rows, size_t o0, size_t o1, float* y) {
    return gemv_ws_level(0, ty, w, n_out, k, ws, xf, rows, o0, o1, y);
}

int or_gemv(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows,
            float* y) {
    return or_gemv_threads(ty, w, n_out, k, x, rows, y, 1);
}

/* gemv.rs:402-431 partition and row_align */
void or_partition(int ty, size_t n_out, size_t k, size_t parts, size_t* starts, size_t* ends) {
    if (parts == 0) parts = 1;
    size_t row_bytes = k / (size_t)or_block_elems(ty) * (size_t)or_block_bytes(ty);
    size_t align = 1;
    for (size_t r = 1; r <= 8; ++r)
        if ((r * row_bytes) % 64 == 0) {
            align = r;
            break;
        }
    size_t units = (n_out + align - 1) / align;
    size_t base = units / parts, extra = units % parts;
    for (size_t p = 0; p < parts; ++p) {
        size_t su = p * base + (p < extra ? p : extra);
        size_t eu = su + base + (p < extra ? 1 : 0);
        size_t s = su * align, e = eu * align;
        starts[p] = s < n_out ? s : n_out;
        ends[p] = e < n_out ? e : n_out;
    }
}

struct gemv_job {
    int level, ty;
    const uint8_t* w;
    size_t n_out, k, rows, o0, o1;
    const uint8_t* ws;
    const float* x;
    float* y;
};

static void* gemv_worker(void* p) {
    struct gemv_job* j = (struct gemv_job*)p;
    gemv_ws_level(j->level, j->ty, j->w, j->n_out, j->k, j->ws, j->x, j->rows, j->o0, j->o1, j->y);
    return NULL;
}

static int gemv_threads_level(int level, int ty, const uint8_t* w, size_t n_out, size_t k, const float* x,
                              size_t rows, float* y, int threads);

int or_gemv_threads(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x,
                    size_t rows, float* y, int threads) {
    return gemv_threads_level(0, ty, w, n_out, k, x, rows, y, threads);
}

int or_gemv_x86(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows, float* y,
                int threads) {
    return gemv_threads_level(1, ty, w, n_out, k, x, rows, y, threads);
}

static int gemv_threads_level(int level, int ty, const uint8_t* w, size_t n_out, size_t k, const float* x,
                              size_t rows, float* y, int threads) {
    if (!or_block_elems(ty) || k % (size_t)or_block_elems(ty)) return -1;
    int kind = or_act_kind(ty);
    size_t wsb = or_act_workspace_bytes(kind, rows, k);
    uint8_t* ws = wsb ? (uint8_t*)malloc(wsb) : NULL;
    if (wsb && !ws) return -1;
    if (kind != OR_ACT_F32 && or_act_quantize(kind, x, rows, k, ws)) {
        free(ws);
        return -1;
    }
    if (threads < 1) threads = 1;
    if (threads == 1) {
        int rc = gemv_ws_level(level, ty, w, n_out, k, ws, x, rows, 0, n_out, y);
        free(ws);
        return rc;
    }
    size_t* st = (size_t*)calloc((size_t)threads * 2, sizeof(size_t));
    struct gemv_job* jobs = (struct gemv_job*)calloc((size_t)threads, sizeof *jobs);
    pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof *tid);
    or_partition(ty, n_out, k, (size_t)threads, st, st + threads);
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (struct gemv_job){level, ty, w, n_out, k, rows, st[t], st[threads + t], ws, x, y};
        pthread_create(&tid[t], NULL, gemv_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(tid);
    free(jobs);
    free(st);
    free(ws);
    return 0;
}

/* ===================================================================================== */
/* GateUpAct{Silu} on quantized weights.  kernels::reference defines the op as               */
/* y[r][i] = silu(gate_i . x_r) * (up_i . x_r) (crates/kernels/src/reference/linear.rs:75-112); */
/* the ggml provider binds one weight of 2 n_out rows, gate rows first, then up rows          */
/* (crates/kernels-ggml/src/mapping.rs:31).  On quantized weights each dot is the Gemv value */
/* and the gated product is the MoE FFN's (crates/kernels-cpu/src/moe.rs:529-551): silu with  */
/* the software exp, the product rounded once.                                              */
/* ===================================================================================== */

/* ===================================================================================== */
/* RmsNorm and Logits: crates/kernels/src/reference/norm.rs:39-47 (Norm::row) and           */
/* crates/kernels/src/reference/linear.rs:118-161 (logits: each row normalised, then the head */
/* as Gemv).  The head product is the CPU provider's Gemv (or_gemv), as a provider computes */
/* its Gemv-class ops.                                                                        */
/* ===================================================================================== */

/* ss = sum of x[i] x[i] in the F32Fixed order; mean = ss / n; scale = 1 / sqrt(mean + eps);
 * y[i] = (x[i] scale) g[i]: each step one IEEE F32 operation */
void or_rms_norm_row(const float* x, const float* g, size_t n, float eps, float* y) {
    const float ss = or_dot(x, x, n);
    const float mean = ss / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; ++i) y[i] = (x[i] * scale) * g[i];
}

int or_rms_norm(const float* x, const float* g, size_t rows, size_t n, float eps, float* y) {
    if (n == 0) return 0;
    for (size_t r = 0; r < rows; ++r) or_rms_norm_row(x + r * n, g, n, eps, y + r * n);
    return 0;
}

int or_logits(int ty, const uint8_t* head, size_t vocab, size_t hidden, const float* g, float eps,
              const float* x, size_t rows, float* y, int threads) {
    float* h = (float*)malloc(rows * hidden * sizeof(float) + 1);
    if (!h) return -1;
    or_rms_norm(x, g, rows, hidden, eps, h);
    const int rc = or_gemv_threads(ty, head, vocab, hidden, h, rows, y, threads);
    free(h);
    return rc;
}

int or_gate_up_act(int ty, const uint8_t* w, size_t n_out, size_t k, const float* x, size_t rows,
                   float* y, int threads) {
    float* y2 = (float*)malloc(rows * 2 * n_out * sizeof(float) + 1);
    if (!y2) return -1;
    int rc = or_gemv_threads(ty, w, 2 * n_out, k, x, rows, y2, threads);
    if (!rc)
        for (size_t r = 0; r < rows; ++r)
            for (size_t i = 0; i < n_out; ++i)
                y[r * n_out + i] = or_silu(y2[r * 2 * n_out + i]) * y2[r * 2 * n_out + n_out + i];
    free(y2);
    return rc;
}

/* ===================================================================================== */
/* MoeGrouped: crates/kernels-cpu/src/moe.rs:402-551                                       */
/* ===================================================================================== */

static size_t act_bytes_max(size_t rows, size_t k) {
    size_t a = or_act_workspace_bytes(OR_ACT_Q8_0, rows, k);
    size_t b = or_act_workspace_bytes(OR_ACT_Q8K, rows, k);
    return a > b ? a : b;
}
static size_t round4(size_t v) { return (v + 3) / 4 * 4; }

/* moe.rs:302-308 workspace_bytes */
size_t or_moe_workspace_bytes(size_t n_experts, size_t top_k, size_t hidden, size_t inter,
                              size_t rows) {
    size_t words = (n_experts + 1) + rows * top_k;
    size_t f32s = rows * hidden + 2 * rows * inter + rows * hidden;
    size_t acts = round4(act_bytes_max(rows, hidden)) + round4(act_bytes_max(rows, inter));
    return 4 + 4 * (words + f32s) + acts;
}

/* moe.rs:431-457: counting sort of slots r*top_k+j by expert, stable in slot order */
int or_moe_pack(const int32_t* ids, size_t rows, size_t top_k, size_t n_experts,
                uint32_t* offsets, uint32_t* slots) {
    size_t n = rows * top_k;
    for (size_t e = 0; e <= n_experts; ++e) offsets[e] = 0;
    for (size_t s = 0; s < n; ++s) {
        if (ids[s] < 0 || (size_t)ids[s] >= n_experts) return -1;
        offsets[ids[s] + 1] += 1;
    }
    for (size_t e = 0; e < n_experts; ++e) offsets[e + 1] += offsets[e];
    for (size_t s = 0; s < n; ++s) {
        size_t e = (size_t)ids[s];
        slots[offsets[e]] = (uint32_t)s;
        offsets[e] += 1;
    }
    for (size_t e = n_experts; e >= 1; --e) offsets[e] = offsets[e - 1];
    offsets[0] = 0;
    return 0;
}

struct moe_ctx {
    int gate_ty, down_ty;
    size_t n_experts, top_k, hidden, inter, rows;
    const uint8_t *gate, *up, *down;
    const float* x;
    const int32_t* site;
    float* out;
    const uint32_t *offsets, *slots;
    size_t e_begin, e_end, stride; /* experts e_begin, e_begin+stride, ... */
    int level;                     /* the Gemv kernels' level (gemv_ws_level) */
};

/* moe.rs:470-517: one expert's pass: gather distinct rows, quantize, gate/up + silu, requant h,
 * down, scatter to every slot of the row */
static int moe_expert(const struct moe_ctx* c, size_t e, float* xg, float* g, float* u, float* yd,
                      uint8_t* xq, uint8_t* hq) {
    size_t g0 = c->offsets[e], g1 = c->offsets[e + 1];
    size_t H = c->hidden, I = c->inter, K = c->top_k;
    size_t gbytes = I * (H / (size_t)or_block_elems(c->gate_ty)) * (size_t)or_block_bytes(c->gate_ty);
    size_t dbytes = H * (I / (size_t)or_block_elems(c->down_ty)) * (size_t)or_block_bytes(c->down_ty);
    const uint8_t* gw = c->gate + e * gbytes;
    const uint8_t* uw = c->up + e * gbytes;
    const uint8_t* dw = c->down + e * dbytes;
    size_t n = 0;
    for (size_t i = g0; i < g1; ++i) {
        size_t r = c->slots[i] / K;
        if (i > g0 && c->slots[i - 1] / K == r) continue;
        memcpy(xg + n * H, c->x + r * H, H * 4);
        n++;
    }
    if (or_act_quantize(or_act_kind(c->gate_ty), xg, n, H, xq)) return -1;
    gemv_ws_level(c->level, c->gate_ty, gw, I, H, xq, xg, n, 0, I, g);
    gemv_ws_level(c->level, c->gate_ty, uw, I, H, xq, xg, n, 0, I, u);
    for (size_t i = 0; i < n * I; ++i) g[i] = or_silu(g[i]) * u[i];
    if (or_act_quantize(or_act_kind(c->down_ty), g, n, I, hq)) return -1;
    gemv_ws_level(c->level, c->down_ty, dw, H, I, hq, g, n, 0, H, yd);
    size_t row_i = 0;
    for (size_t i = g0; i < g1; ++i) {
        size_t r = c->slots[i] / K;
        if (i > g0 && c->slots[i - 1] / K != r) row_i++;
        memcpy(c->out + (size_t)c->slots[i] * H, yd + row_i * H, H * 4);
    }
    return 0;
}

static void* moe_worker(void* p) {
    const struct moe_ctx* c = (const struct moe_ctx*)p;
    size_t H = c->hidden, I = c->inter, R = c->rows;
    float* xg = (float*)malloc(R * H * 4);
    float* g = (float*)malloc(R * I * 4);
    float* u = (float*)malloc(R * I * 4);
    float* yd = (float*)malloc(R * H * 4);
    uint8_t* xq = (uint8_t*)malloc(act_bytes_max(R, H) + 4);
    uint8_t* hq = (uint8_t*)malloc(act_bytes_max(R, I) + 4);
    for (size_t e = c->e_begin; e < c->e_end; e += c->stride) {
        if (c->offsets[e] == c->offsets[e + 1]) continue;
        if (c->site && !c->site[e]) continue;
        moe_expert(c, e, xg, g, u, yd, xq, hq);
    }
    free(xg); free(g); free(u); free(yd); free(xq); free(hq);
    return NULL;
}

static int moe_grouped_level(int level, int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                             size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                             const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                             float* out, int threads);

int or_moe_grouped(int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                   size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                   const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                   float* out, int threads) {
    return moe_grouped_level(0, gate_ty, down_ty, n_experts, top_k, hidden, inter, gate, up, down, x, ids, site,
                             rows, out, threads);
}

int or_moe_grouped_x86(int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                       size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                       float* out, int threads) {
    return moe_grouped_level(1, gate_ty, down_ty, n_experts, top_k, hidden, inter, gate, up, down, x, ids, site,
                             rows, out, threads);
}

static int moe_grouped_level(int level, int gate_ty, int down_ty, size_t n_experts, size_t top_k, size_t hidden,
                             size_t inter, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                             const float* x, const int32_t* ids, const int32_t* site, size_t rows,
                             float* out, int threads) {
    if ((gate_ty != OR_Q4_K && gate_ty != OR_Q8_0) || (down_ty != OR_Q4_K && down_ty != OR_Q8_0))
        return -1;
    if (hidden % (size_t)or_block_elems(gate_ty) || inter % (size_t)or_block_elems(down_ty))
        return -1;
    if (rows == 0) return 0;
    uint32_t* offsets = (uint32_t*)malloc((n_experts + 1) * 4);
    uint32_t* slots = (uint32_t*)malloc(rows * top_k * 4);
    if (or_moe_pack(ids, rows, top_k, n_experts, offsets, slots)) {
        free(offsets);
        free(slots);
        return -2;
    }
    if (threads < 1) threads = 1;
    struct moe_ctx base = {gate_ty, down_ty, n_experts, top_k, hidden, inter, rows, gate, up,
                           down, x, site, out, offsets, slots, 0, n_experts, 1, level};
    if (threads == 1) {
        moe_worker(&base);
    } else {
        /* experts split across threads (moe.rs:46-51: tasks of distinct experts are
         * independent); expert e goes to thread e mod threads */
        pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof *tid);
        struct moe_ctx* cs = (struct moe_ctx*)calloc((size_t)threads, sizeof *cs);
        for (int t = 0; t < threads; ++t) {
            cs[t] = base;
            cs[t].e_begin = (size_t)t;
            cs[t].stride = (size_t)threads;
            pthread_create(&tid[t], NULL, moe_worker, &cs[t]);
        }
        for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
        free(tid);
        free(cs);
    }
    free(offsets);
    free(slots);
    return 0;
}

/* ===================================================================================== */
/* MoeRoute{Softmax}: no reference code.  Specification followed:                          */
/*   logits in F32 as F32Fixed dots (RFC-0040 §3 fixed-order rule, ...md:294,848;           */
/*   reduce.rs:30-90); softmax F32Fixed: subtract the row max (reference.rs:56-59), software */
/*   exp (math.rs:45-75), F32Fixed sum, one division per element; top-k on the F32          */
/*   probabilities, ties to the lower expert index (RFC-0042 ...md:232); renormalize       */
/*   (graph/src/blocks/ffn.rs:145-146) divides each selected probability by the F32Fixed     */
/*   sum of the k selected probabilities in rank order.                                     */
/* ===================================================================================== */

int or_moe_route(const float* router, const float* x, size_t rows, size_t hidden,
                 size_t n_experts, size_t top_k, int renormalize, int32_t* ids, float* weights,
                 float* probs) {
    if (top_k == 0 || top_k > n_experts || top_k > 64) return -1;
    float* p = (float*)malloc(n_experts * 4);
    unsigned char* taken = (unsigned char*)malloc(n_experts);
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * hidden;
        for (size_t e = 0; e < n_experts; ++e) p[e] = or_dot(router + e * hidden, xr, hidden);
        float m = p[0];
        for (size_t e = 1; e < n_experts; ++e)
            if (p[e] > m) m = p[e];
        for (size_t e = 0; e < n_experts; ++e) p[e] = or_exp(p[e] - m);
        float s = or_sum(p, n_experts);
        for (size_t e = 0; e < n_experts; ++e) p[e] = p[e] / s;
        if (probs) memcpy(probs + r * n_experts, p, n_experts * 4);
        memset(taken, 0, n_experts);
        float sel[64];
        for (size_t j = 0; j < top_k; ++j) {
            size_t best = n_experts;
            for (size_t e = 0; e < n_experts; ++e) {
                if (taken[e]) continue;
                if (best == n_experts || p[e] > p[best]) best = e;
            }
            taken[best] = 1;
            ids[r * top_k + j] = (int32_t)best;
            sel[j] = p[best];
        }
        if (renormalize) {
            float t = or_sum(sel, top_k);
            for (size_t j = 0; j < top_k; ++j) weights[r * top_k + j] = sel[j] / t;
        } else {
            for (size_t j = 0; j < top_k; ++j) weights[r * top_k + j] = sel[j];
        }
    }
    free(p);
    free(taken);
    return 0;
}

/* ===================================================================================== */
/* MoeCombine: crates/kernels-cpu/src/moe/tests.rs:541-556 (the helper is its only code)   */
/* per row: slots in ascending expert id (stable), y += w * v in F32 from 0.0, no FMA.     */
/* ===================================================================================== */

int or_moe_combine(const float* out, const int32_t* ids, const float* w, size_t rows,
                   size_t top_k, size_t hidden, float* y) {
    if (top_k > 64) return -1;
    for (size_t r = 0; r < rows; ++r) {
        size_t order[64];
        for (size_t j = 0; j < top_k; ++j) order[j] = j;
        /* stable insertion sort by id */
        for (size_t a = 1; a < top_k; ++a) {
            size_t v = order[a], b = a;
            while (b > 0 && ids[r * top_k + order[b - 1]] > ids[r * top_k + v]) {
                order[b] = order[b - 1];
                b--;
            }
            order[b] = v;
        }
        float* yr = y + r * hidden;
        for (size_t i = 0; i < hidden; ++i) yr[i] = 0.0f;
        for (size_t a = 0; a < top_k; ++a) {
            size_t j = order[a];
            const float* slot = out + (r * top_k + j) * hidden;
            float wj = w[r * top_k + j];
            for (size_t i = 0; i < hidden; ++i) yr[i] += wj * slot[i];
        }
    }
    return 0;
}

/* ===================================================================================== */
/* MoeCombine as the IR binds it: inputs [per_expert, weights, shared...], dims            */
/* [top_k, n_shared, hidden] (crates/kernels/src/op/kind.rs:244;                           */
/* crates/graph/src/ir/signature.rs:153; crates/graph/src/blocks/ffn.rs:189-200).  The      */
/* binding carries no expert ids, so the routed slots are added in rank order, as          */
/* plan/rfcs/RFC-0042-quantization-and-numerical-fidelity.md:233 states (slot j = rank j),  */
/* then the shared experts' outputs in input order (RFC-0040 ...md:296): y = 0.0,          */
/* y += w_j * v_j (product rounded, then the sum), y += shared_s, in F32, no FMA.          */
/* shared: n_shared arrays of [rows, hidden], contiguous ([n_shared][rows][hidden]).        */
/* ===================================================================================== */

int or_moe_combine_ranked(const float* out, const float* w, const float* shared, size_t n_shared,
                          size_t rows, size_t top_k, size_t hidden, float* y) {
    for (size_t r = 0; r < rows; ++r) {
        float* yr = y + r * hidden;
        for (size_t i = 0; i < hidden; ++i) yr[i] = 0.0f;
        for (size_t j = 0; j < top_k; ++j) {
            const float* slot = out + (r * top_k + j) * hidden;
            const float wj = w[r * top_k + j];
            for (size_t i = 0; i < hidden; ++i) yr[i] += wj * slot[i];
        }
        for (size_t s = 0; s < n_shared; ++s) {
            const float* sh = shared + (s * rows + r) * hidden;
            for (size_t i = 0; i < hidden; ++i) yr[i] += sh[i];
        }
    }
    return 0;
}

/* ===================================================================================== */
/* Seeded synthetic data and helpers                                                       */
/* ===================================================================================== */

static inline uint64_t splitmix64(uint64_t* s) {
    *s += 0x9E3779B97F4A7C15ull;
    uint64_t z = *s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* SplitMix64 -> two uniforms -> Box-Muller in F64 -> x sigma -> F32 */
void or_normal_f32(uint64_t seed, float sigma, float* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2) * (double)sigma);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2) * (double)sigma);
    }
}

uint64_t or_fnv1a(const uint8_t* bytes, size_t n) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (size_t i = 0; i < n; ++i) h = (h ^ bytes[i]) * 0x00000100000001B3ull;
    return h;
}

int or_num_threads_default(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

/* ============================================================================================
 * The residency split
 * ========================================================================================== */

/* Stable merge sort of miss indices by tokens descending, then expert ascending. */
static int miss_before(const struct or_route_slot* r, uint32_t a, uint32_t b) {
    if (r[a].tokens != r[b].tokens) return r[a].tokens > r[b].tokens;
    return r[a].expert < r[b].expert;
}
static void sort_misses(const struct or_route_slot* r, uint32_t* v, uint32_t* tmp, uint32_t n) {
    for (uint32_t w = 1; w < n; w *= 2) {
        for (uint32_t lo = 0; lo < n; lo += 2 * w) {
            uint32_t mid = lo + w < n ? lo + w : n, hi = lo + 2 * w < n ? lo + 2 * w : n;
            uint32_t i = lo, j = mid, k = lo;
            /* the left run wins ties: stable */
            while (i < mid && j < hi) tmp[k++] = miss_before(r, v[j], v[i]) ? v[j++] : v[i++];
            while (i < mid) tmp[k++] = v[i++];
            while (j < hi) tmp[k++] = v[j++];
        }
        memcpy(v, tmp, (size_t)n * 4);
    }
}

/* RFC-0040 ...md:392-403 (RFC-0023 section 6), the split function as written there: the misses
 * ordered by tokens descending, then expert index ascending (entries of one expert, which a
 * well-formed doorbell never repeats, in entry order), walked; a miss marked in the eligibility
 * bitmap (bit e % 32 of word e / 32, for e below n_experts) is copied while its bytes keep the
 * copied total at or below b_copy and a copy slot is left, taking the next copy-slot index;
 * hits are HIT, every other miss CPU.  The doc of crates/kernels/src/moe.rs:110-125 states the
 * same rule. */
void or_moe_assign(const struct or_route_slot* route, uint32_t n_route, const uint32_t* eligible,
                   uint32_t n_experts, uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots,
                   uint32_t* out) {
    uint32_t* miss = (uint32_t*)malloc((size_t)(n_route + 1) * 4);
    uint32_t* tmp = (uint32_t*)malloc((size_t)(n_route + 1) * 4);
    uint32_t m = 0;
    for (uint32_t i = 0; i < n_route; ++i) {
        if (route[i].cache_slot != OR_MOE_MISS) {
            out[i] = OR_MOE_HIT;
        } else {
            out[i] = OR_MOE_CPU;
            miss[m++] = i;
        }
    }
    sort_misses(route, miss, tmp, m);
    uint32_t copied = 0;
    uint64_t bytes = 0; /* never above b_copy */
    for (uint32_t t = 0; t < m; ++t) {
        const uint32_t i = miss[t], e = route[i].expert;
        const int marked = e < n_experts && ((eligible[e / 32] >> (e % 32)) & 1u);
        const int fits = expert_bytes <= (uint64_t)b_copy - bytes;
        if (marked && fits && copied < copy_slots) {
            out[i] = copied++;
            bytes += expert_bytes;
        }
    }
    free(miss);
    free(tmp);
}

/* RFC-0040 ...md:390 and RFC-0023 section 2: the router op's doorbell layer, the step's seq, then
 * one RouteSlot { expert, tokens, cache_slot } per distinct expert the pass selected, tokens the
 * rows that selected it; n_pred = 0 (no predictions), the pred part untouched.  Entries are in
 * ascending expert index (the split rule does not depend on their order,
 * crates/kernels/src/moe/tests.rs:612-627).  Layout: moe_doorbell.h, little-endian. */
int or_moe_doorbell(const int32_t* ids, size_t rows, size_t top_k, uint32_t n_experts,
                    const uint32_t* slot_of, uint32_t seq, uint32_t max_union, uint8_t* layer) {
    uint32_t* cnt = (uint32_t*)calloc((size_t)n_experts + 1, 4);
    for (size_t r = 0; r < rows; ++r) {
        for (size_t j = 0; j < top_k; ++j) {
            const int32_t e = ids[r * top_k + j];
            if (e < 0 || (uint32_t)e >= n_experts) {
                free(cnt);
                return -1;
            }
            int again = 0;
            for (size_t q = 0; q < j; ++q) again |= ids[r * top_k + q] == e;
            if (!again) cnt[e] += 1;
        }
    }
    uint32_t n = 0;
    for (uint32_t e = 0; e < n_experts; ++e) n += cnt[e] != 0;
    if (n > max_union) {
        free(cnt);
        return -2;
    }
    const uint16_t n_route = (uint16_t)n, n_pred = 0;
    memcpy(layer + 0, &seq, 4);
    memcpy(layer + 4, &n_route, 2);
    memcpy(layer + 6, &n_pred, 2);
    uint32_t i = 0;
    for (uint32_t e = 0; e < n_experts; ++e) {
        if (!cnt[e]) continue;
        const uint16_t ex = (uint16_t)e, tok = (uint16_t)cnt[e];
        const uint32_t slot = slot_of ? slot_of[e] : OR_MOE_MISS;
        uint8_t* p = layer + 8 + 8 * (size_t)i++;
        memcpy(p + 0, &ex, 2);
        memcpy(p + 2, &tok, 2);
        memcpy(p + 4, &slot, 4);
    }
    free(cnt);
    return 0;
}
