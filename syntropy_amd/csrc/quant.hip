// Weight quantizers and exact dequantizers on gfx950.
//
// The quantizers follow ggml (Copyright (c) 2023-2026 The ggml authors, MIT License; the notice
// is in THIRD_PARTY.md at the repository root).
//
// The quantizers are ggml's reference routines (third_party/ggml/src/ggml-quants.c:113-140
// quantize_row_q4_0_ref, :276-297 quantize_row_q8_0_ref, :799-878 make_qkx2_quants,
// :1458-1528 quantize_row_q4_K_ref), one block per thread, operation for operation: every
// float operation is one IEEE F32 operation (no contraction, correctly rounded division and
// square root), so the bytes equal ggml's.  The dequantizers are
// crates/kernels/src/reference/dequant.rs:133-173.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

SYN_DEV void put16(uint8_t* p, uint32_t h) {
    p[0] = (uint8_t)h;
    p[1] = (uint8_t)(h >> 8);
}

__global__ __launch_bounds__(256) void k_quantize_q4_0(const float* __restrict__ xall,
                                                       uint8_t* __restrict__ y, uint64_t nb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb) return;
    const float* x = xall + i * 32;
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float v = x[j];
        if (amax < __builtin_fabsf(v)) {
            amax = __builtin_fabsf(v);
            mx = v;
        }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* blk = y + i * 18;
    put16(blk, f16_bits(d));
    for (int j = 0; j < 16; ++j) {
        const float x0 = x[j] * id;
        const float x1 = x[16 + j] * id;
        const int t0 = (int)(int8_t)(int)(x0 + 8.5f);
        const int t1 = (int)(int8_t)(int)(x1 + 8.5f);
        const int xi0 = t0 < 15 ? t0 : 15;
        const int xi1 = t1 < 15 ? t1 : 15;
        blk[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ xall,
                                                       uint8_t* __restrict__ y, uint64_t nb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb) return;
    const float* x = xall + i * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = __builtin_fabsf(x[j]);
        amax = amax > a ? amax : a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* blk = y + i * 34;
    put16(blk, f16_bits(d));
    for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)(int)__builtin_roundf(x[j] * id);
}

// make_qkx2_quants with nmax 15, rmin -1, rdelta 0.1, nstep 20, use_mad false.
SYN_DEV float make_qkx2(const float* x, const float* weights, uint8_t* L, float* the_min) {
    const int n = 32, nmax = 15, nstep = 20;
    const float rmin = -1.f, rdelta = 0.1f;
    uint8_t Laux[32];
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = (float)nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        l = l < nmax ? l : nmax;
        L[i] = (uint8_t)(l > 0 ? l : 0);
        float diff = scale * (float)L[i] + min - x[i];
        diff = diff * diff;
        best_error += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < nmax ? l : nmax;
            l = l > 0 ? l : 0;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            const float lf = (float)l;
            sum_l += w * lf;
            sum_l2 += w * lf * lf;
            sum_xl += w * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += weights[i] * diff;
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

__global__ __launch_bounds__(64) void k_quantize_q4_k(const float* __restrict__ xall,
                                                      uint8_t* __restrict__ y, uint64_t nb) {
    const uint64_t i = (uint64_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= nb) return;
    const float* x = xall + i * 256;
    uint8_t L[256];
    float weights[32];
    float mins[8], scales[8];
    uint8_t sc12[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = __builtin_sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + __builtin_fabsf(x[32 * j + l]);
        scales[j] = make_qkx2(x + 32 * j, weights, L + 32 * j, &mins[j]);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (j < 4) {
            sc12[j] = ls;
            sc12[j + 4] = lm;
        } else {
            sc12[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc12[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc12[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint32_t dh = f16_bits(max_scale / 63.f);
    const uint32_t mh = f16_bits(max_min / 63.f);
    const float dd = f16_to_f32(dh), dm16 = f16_to_f32(mh);
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        if (j < 4) {
            sc = sc12[j] & 63;
            m = sc12[j + 4] & 63;
        } else {
            sc = (sc12[j + 4] & 0xF) | ((sc12[j - 4] >> 6) << 4);
            m = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
        }
        const float d = dd * (float)sc;
        if (!(d != 0.0f)) continue;
        const float dm = dm16 * (float)m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            l = l < 15 ? l : 15;
            l = l > 0 ? l : 0;
            L[32 * j + ii] = (uint8_t)l;
        }
    }
    uint8_t* blk = y + i * 144;
    put16(blk, dh);
    put16(blk + 2, mh);
    for (int j = 0; j < 12; ++j) blk[4 + j] = sc12[j];
    for (int jj = 0; jj < 4; ++jj)
        for (int l = 0; l < 32; ++l)
            blk[16 + 32 * jj + l] = (uint8_t)(L[64 * jj + l] | (L[64 * jj + l + 32] << 4));
}

// Exact dequantization, one block per thread (dequant.rs:133-173).
__global__ __launch_bounds__(256) void k_dequantize(int ty, const uint8_t* __restrict__ src,
                                                    float* __restrict__ out, uint64_t nb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb) return;
    if (ty == T_Q8_0) {
        const uint8_t* b = src + i * 34;
        const float d = f16_to_f32(b[0] | (b[1] << 8));
        for (int j = 0; j < 32; ++j) out[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
    } else if (ty == T_Q4_0) {
        const uint8_t* b = src + i * 18;
        const float d = f16_to_f32(b[0] | (b[1] << 8));
        for (int j = 0; j < 16; ++j) {
            out[i * 32 + j] = (float)((int)(b[2 + j] & 0xF) - 8) * d;
            out[i * 32 + 16 + j] = (float)((int)(b[2 + j] >> 4) - 8) * d;
        }
    } else if (ty == T_Q4_K) {
        const uint8_t* b = src + i * 144;
        const float d = f16_to_f32(b[0] | (b[1] << 8));
        const float mn = f16_to_f32(b[2] | (b[3] << 8));
        uint32_t w[3];
        for (int t = 0; t < 3; ++t)
            w[t] = b[4 + 4 * t] | (b[5 + 4 * t] << 8) | (b[6 + 4 * t] << 16) | ((uint32_t)b[7 + 4 * t] << 24);
        int sc[8], m[8];
        scales_k4(w[0], w[1], w[2], sc, m);
        for (int g = 0; g < 4; ++g) {
            const float d1 = d * (float)sc[2 * g], m1 = mn * (float)m[2 * g];
            const float d2 = d * (float)sc[2 * g + 1], m2 = mn * (float)m[2 * g + 1];
            for (int l = 0; l < 32; ++l) {
                const uint8_t q = b[16 + 32 * g + l];
                out[i * 256 + 64 * g + l] = d1 * (float)(q & 0xF) - m1;
                out[i * 256 + 64 * g + 32 + l] = d2 * (float)(q >> 4) - m2;
            }
        }
    }
}

void launch_quantize(int ty, const float* x, uint64_t n, uint8_t* out, hipStream_t stream) {
    const uint64_t nb = n / (uint64_t)block_elems(ty);
    if (nb == 0) return;
    if (ty == T_Q4_0)
        hipLaunchKernelGGL(k_quantize_q4_0, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0,
                           stream, x, out, nb);
    else if (ty == T_Q8_0)
        hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0,
                           stream, x, out, nb);
    else if (ty == T_Q4_K)
        hipLaunchKernelGGL(k_quantize_q4_k, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, stream,
                           x, out, nb);
}

void launch_dequantize(int ty, const uint8_t* src, uint64_t n, float* out, hipStream_t stream) {
    const uint64_t nb = n / (uint64_t)block_elems(ty);
    if (nb == 0) return;
    hipLaunchKernelGGL(k_dequantize, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream, ty,
                       src, out, nb);
}

}  // namespace syn
