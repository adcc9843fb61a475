// Decode GEMV over GGUF Q4_0 / Q8_0 / Q4_K weights on gfx950.
//
// Value: crates/kernels-cpu/src/gemv.rs:1-60 and gemv/portable.rs:114-190.  Per output row and
// activation row, each weight block gives one exact I32 block sum and one F32 term
// (q32_term / q4k_term, gemv.rs:539-547), and the terms are added in ascending block order
// into an F32 accumulator that starts at +0.0.  The kernels reproduce that value bit for bit.
//
// Mapping.  A wavefront owns G = 64/P output rows; the P lanes of a row take the row's blocks
// in turn (block b -> lane b mod P), so a row's terms are produced P at a time and folded in
// order by handing the running sum from lane to lane with a DPP rotation.  Weight bytes are
// streamed with 16-byte loads into a per-wavefront LDS stage (G row segments of C blocks),
// then each lane reads its own block back from LDS: the global reads are contiguous and the
// LDS reads (a 144- or 136-byte lane stride) are bank-conflict free.  Quantized activations
// are read from the workspace (they stay in L1/L2); up to R = 8 activation rows share each
// decoded weight block.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

template <int FMT>
struct Fmt;
template <>
struct Fmt<T_Q4_K> {
    static constexpr int BB = 144, BE = 256, U = 1;
};
template <>
struct Fmt<T_Q4_0> {
    static constexpr int BB = 18, BE = 32, U = 8;
};
template <>
struct Fmt<T_Q8_0> {
    static constexpr int BB = 34, BE = 32, U = 4;
};

template <int FMT, int P>
struct Geo {
    static constexpr int G = 64 / P;                   // rows per wavefront
    static constexpr int C = P * Fmt<FMT>::U;           // blocks per row per stage
    static constexpr int SEG = C * Fmt<FMT>::BB;        // bytes per row per stage
    static constexpr int STAGE = G * SEG + 64;          // + slack for the over-reads
};

struct ActPtrs {
    const int8_t* q;
    const float* d;
    const int32_t* s;
    int64_t k;  // values per activation row
};

template <int VEC>
SYN_DEV void copy_piece(uint8_t* dst, const uint8_t* src) {
    if constexpr (VEC == 16) {
        typedef unsigned int v4u __attribute__((ext_vector_type(4)));
        *reinterpret_cast<v4u*>(dst) = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src));
    } else {
        *dst = *src;
    }
}

// Term of one Q4_K super-block for activation row r (crates/kernels-cpu/src/gemv.rs:539-547,
// portable.rs:97-110, 157-185).
SYN_DEV float q4k_term(const uint32_t* wb, const ActPtrs& a, int r, int64_t b) {
    int sc[8], mn[8];
    scales_k4(wb[1], wb[2], wb[3], sc, mn);
    const float d = f16_to_f32(wb[0]);
    const float dmin = f16_to_f32(wb[0] >> 16);
    const uint4* xv = reinterpret_cast<const uint4*>(a.q + r * a.k + b * 256);
    const int4* xs4 = reinterpret_cast<const int4*>(a.s + (r * a.k + b * 256) / 32);
    const float dx = a.d[(r * a.k) / 256 + b];
    int s1 = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 xl0 = xv[4 * g + 0], xl1 = xv[4 * g + 1];
        const uint4 xh0 = xv[4 * g + 2], xh1 = xv[4 * g + 3];
        const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t q = wb[4 + 8 * g + t];
            lo = sdot4(q & 0x0F0F0F0Fu, xl[t], lo);
            hi = sdot4((q >> 4) & 0x0F0F0F0Fu, xh[t], hi);
        }
        s1 = mad24(sc[2 * g + 1], hi, mad24(sc[2 * g], lo, s1));
    }
    const int4 sa = xs4[0], sb = xs4[1];
    const int s2 = q4k_s2(mn, sa, sb);
    return (d * dx) * (float)s1 - (dmin * dx) * (float)s2;
}

// Term of one 32-value block (Q4_0 or Q8_0) for activation row r: (dw*dx)*s.
template <int FMT>
SYN_DEV float q32_term(uint32_t dw16, const uint32_t* qs, const ActPtrs& a, int r, int64_t b) {
    const uint4* xv = reinterpret_cast<const uint4*>(a.q + r * a.k + b * 32);
    const uint4 x0 = xv[0], x1 = xv[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const int64_t bi = (r * a.k) / 32 + b;
    int s = 0;
    if constexpr (FMT == T_Q4_0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s = sdot4(qs[t] & 0x0F0F0F0Fu, xw[t], s);
            s = sdot4((qs[t] >> 4) & 0x0F0F0F0Fu, xw[t + 4], s);
        }
        s -= 8 * a.s[bi];  // (n - 8) codes: sum n*x - 8 * sum x, exact
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) s = sdot4(qs[t], xw[t], s);
    }
    return (f16_to_f32(dw16) * a.d[bi]) * (float)s;
}

template <int FMT, int P, int R, int VEC>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ W, int n_out, int nb,
                                              int64_t row_bytes, ActPtrs act, int rows,
                                              float* __restrict__ y, int64_t y_stride,
                                              const uint32_t* __restrict__ active, int first) {
    rows = active_rows(active, first, rows);
    if (rows == 0) return;  // uniform
    using F = Fmt<FMT>;
    using Gm = Geo<FMT, P>;
    constexpr int G = Gm::G, C = Gm::C, BB = F::BB;
    __shared__ __attribute__((aligned(16))) uint8_t stage_all[4][Gm::STAGE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint8_t* stage = stage_all[wave];
    const int g = lane / P, j = lane % P;
    const int row0 = (blockIdx.x * 4 + wave) * G;
    const int row = row0 + g;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int cb = 0; cb < nb; cb += C) {
        const int nblk = nb - cb < C ? nb - cb : C;
        const int seg = nblk * BB;
        // Stage G row segments, contiguous 16-byte pieces.
        for (int gg = 0; gg < G; ++gg) {
            if (row0 + gg >= n_out) break;
            const uint8_t* src = W + (int64_t)(row0 + gg) * row_bytes + (int64_t)cb * BB;
            uint8_t* dst = stage + gg * Gm::SEG;
            for (int p = lane; p < seg / VEC; p += 64) copy_piece<VEC>(dst + p * VEC, src + p * VEC);
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < F::U; ++u) {
            const int bi = u * P + j;  // block within this stage
            const bool valid = bi < nblk && row < n_out;
            float t[R];
#pragma unroll
            for (int r = 0; r < R; ++r) t[r] = 0.0f;
            if (valid) {
                const int64_t b = cb + bi;
                const uint8_t* blk = stage + g * Gm::SEG + bi * BB;
                if constexpr (FMT == T_Q4_K) {
                    uint32_t wb[36];
                    const uint4* s4 = reinterpret_cast<const uint4*>(blk);
#pragma unroll
                    for (int i = 0; i < 9; ++i) {
                        const uint4 v = s4[i];
                        wb[4 * i] = v.x;
                        wb[4 * i + 1] = v.y;
                        wb[4 * i + 2] = v.z;
                        wb[4 * i + 3] = v.w;
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (r < rows) t[r] = q4k_term(wb, act, r, b);
                } else {
                    constexpr int NW = FMT == T_Q4_0 ? 6 : 10;  // dwords covering the block
                    constexpr int NQ = FMT == T_Q4_0 ? 4 : 8;   // code dwords
                    const int off = bi * BB;                     // 2-byte aligned
                    const uint32_t* base = reinterpret_cast<const uint32_t*>(blk - (off & 2));
                    uint32_t w[NW];
#pragma unroll
                    for (int i = 0; i < NW; ++i) w[i] = base[i];
                    const bool odd = (off & 2) != 0;
                    const uint32_t dw16 = odd ? (w[0] >> 16) : (w[0] & 0xFFFFu);
                    uint32_t qs[NQ];
#pragma unroll
                    for (int i = 0; i < NQ; ++i) {
                        const uint32_t lo = odd ? w[i + 1] : w[i];
                        const uint32_t hi = odd ? w[i + 2] : w[i + 1];
                        qs[i] = __builtin_amdgcn_alignbyte(hi, lo, odd ? 0u : 2u);
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (r < rows) t[r] = q32_term<FMT>(dw16, qs, act, r, b);
                }
            }
            // In-order fold: the running sum visits the P lanes of the row in turn.
#pragma unroll
            for (int s = 0; s < P; ++s) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r] = rot1<P>(acc[r]);
                    acc[r] = acc[r] + ((j == s) ? t[r] : 0.0f);
                }
            }
        }
        __syncthreads();
    }
    if (j == P - 1 && row < n_out) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < rows) y[r * y_stride + row] = acc[r];
    }
}

template <int FMT, int P, int R>
static void launch_fmt(const uint8_t* W, int n_out, int k, const ActPtrs& a, int rows, float* y,
                       int64_t y_stride, const uint32_t* active, int first, hipStream_t stream) {
    const int nb = k / Fmt<FMT>::BE;
    const int64_t row_bytes = (int64_t)nb * Fmt<FMT>::BB;
    constexpr int G = Geo<FMT, P>::G;
    const dim3 grid((unsigned)((n_out + 4 * G - 1) / (4 * G)));
    const bool vec16 = (row_bytes % 16 == 0) && ((uintptr_t)W % 16 == 0);
    if (vec16)
        hipLaunchKernelGGL((k_gemv<FMT, P, R, 16>), grid, dim3(256), 0, stream, W, n_out, nb,
                           row_bytes, a, rows, y, y_stride, active, first);
    else
        hipLaunchKernelGGL((k_gemv<FMT, P, R, 1>), grid, dim3(256), 0, stream, W, n_out, nb,
                           row_bytes, a, rows, y, y_stride, active, first);
}

template <int FMT, int P>
static void launch_rows(const uint8_t* W, int n_out, int k, const ActPtrs& a, int rows, float* y,
                        int64_t y_stride, const uint32_t* active, int first, hipStream_t stream) {
    if (rows <= 1)
        launch_fmt<FMT, P, 1>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
    else if (rows <= 2)
        launch_fmt<FMT, P, 2>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
    else if (rows <= 4)
        launch_fmt<FMT, P, 4>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
    else
        launch_fmt<FMT, P, 8>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
}

template <int FMT>
static void launch_p(const uint8_t* W, int n_out, int k, const ActPtrs& a, int rows, float* y,
                     int64_t y_stride, const uint32_t* active, int first, hipStream_t stream) {
    const int nb = k / Fmt<FMT>::BE;
    if (nb >= 12)
        launch_rows<FMT, 16>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
    else
        launch_rows<FMT, 4>(W, n_out, k, a, rows, y, y_stride, active, first, stream);
}

// y[r][o] for r < rows, o < n_out, from activations already quantized into `ws` (layout
// act_layout(act_kind(ty), rows, k)).  Rows are taken 8 at a time.
void launch_gemv_q(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int rows,
                   float* y, hipStream_t stream, const uint32_t* active) {
    const ActLayout L = act_layout(act_kind(ty), (uint64_t)rows, (uint64_t)k);
    for (int r0 = 0; r0 < rows; r0 += 8) {
        const int nr = rows - r0 < 8 ? rows - r0 : 8;
        ActPtrs a;
        a.k = k;
        a.q = reinterpret_cast<const int8_t*>(ws + L.codes) + (int64_t)r0 * k;
        a.d = reinterpret_cast<const float*>(ws + L.d) + (int64_t)r0 * (k / block_elems(ty));
        a.s = reinterpret_cast<const int32_t*>(ws + L.sums) + (int64_t)r0 * (k / 32);
        float* yr = y + (int64_t)r0 * n_out;
        switch (ty) {
        case T_Q4_K: launch_p<T_Q4_K>(W, n_out, k, a, nr, yr, n_out, active, r0, stream); break;
        case T_Q4_0: launch_p<T_Q4_0>(W, n_out, k, a, nr, yr, n_out, active, r0, stream); break;
        case T_Q8_0: launch_p<T_Q8_0>(W, n_out, k, a, nr, yr, n_out, active, r0, stream); break;
        default: break;
        }
    }
}

// F16 and BF16 weights (crates/kernels-cpu/src/gemv/portable.rs:30-45 float_rows with the fold
// of gemv.rs:506-516): per output, 32 F32 accumulators; element i goes into accumulator i % 32
// with one fused multiply-add, in increasing i; then the halving fold acc[j] += acc[j + h] for
// h = 16, 8, 4, 2, 1.  Four lanes per weight row: lane j holds accumulators 8j .. 8j + 7 and
// reads the row's elements 32m + 8j .. + 7 (16 bytes, or one element at a time when k is not a
// multiple of 8); 64 rows per workgroup.  Activation rows go FR at a time, each weight chunk
// read once per group.  The activations stay F32 (no quantization).
template <int BF16, int VEC, int FR>
__global__ __launch_bounds__(256) void k_gemv_float(const uint8_t* __restrict__ W, int n_out, int k,
                                                    const float* __restrict__ x, int rows,
                                                    float* __restrict__ y,
                                                    const uint32_t* __restrict__ active) {
    rows = active_rows(active, 0, rows);
    const int j = threadIdx.x & 3;
    const int row = (int)((blockIdx.x * 256u + threadIdx.x) >> 2);
    const bool ok = row < n_out;
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(W + (int64_t)(ok ? row : 0) * k * 2);
    auto cvt = [](uint32_t h) { return BF16 ? __builtin_bit_cast(float, h << 16) : f16_to_f32(h); };
    for (int r0 = 0; r0 < rows; r0 += FR) {  // uniform
        float acc[FR][8];
#pragma unroll
        for (int t = 0; t < FR; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[t][e] = 0.0f;
        for (int i0 = 8 * j; i0 < k; i0 += 32) {
            float w[8];
            if constexpr (VEC) {
                const uint4 v = *reinterpret_cast<const uint4*>(wr + i0);
                const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w[2 * e] = cvt(u[e] & 0xFFFFu);
                    w[2 * e + 1] = cvt(u[e] >> 16);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) w[e] = i0 + e < k ? cvt(wr[i0 + e]) : 0.0f;
            }
#pragma unroll
            for (int t = 0; t < FR; ++t) {
                if (r0 + t >= rows) break;  // uniform
                const float* xr = x + (int64_t)(r0 + t) * k + i0;
                if constexpr (VEC) {
                    const float4 a = reinterpret_cast<const float4*>(xr)[0];
                    const float4 b = reinterpret_cast<const float4*>(xr)[1];
                    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[t][e] = __builtin_fmaf(w[e], xv[e], acc[t][e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (i0 + e < k) acc[t][e] = __builtin_fmaf(w[e], xr[e], acc[t][e]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < FR; ++t) {
            // h = 16: accumulators 8j + e (j < 2) take 8(j + 2) + e; h = 8: lane 0 takes lane 1's
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v16 = __shfl_xor(acc[t][e], 2);
                if (j < 2) acc[t][e] = acc[t][e] + v16;
                const float v8 = __shfl_xor(acc[t][e], 1);
                if (j == 0) acc[t][e] = acc[t][e] + v8;
            }
            // h = 4, 2, 1 inside the lane
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] = acc[t][e] + acc[t][e + 4];
            acc[t][0] = acc[t][0] + acc[t][2];
            acc[t][1] = acc[t][1] + acc[t][3];
            acc[t][0] = acc[t][0] + acc[t][1];
            if (j == 0 && ok && r0 + t < rows) y[(int64_t)(r0 + t) * n_out + row] = acc[t][0];
        }
    }
}

void launch_gemv_float(int ty, const uint8_t* W, int n_out, int k, const float* x, int rows, float* y,
                       hipStream_t stream, const uint32_t* active) {
    const dim3 grid((unsigned)((n_out + 63) / 64));
    const bool vec = k % 8 == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0;
    const bool bf = ty == T_BF16;
    if (vec && bf)
        hipLaunchKernelGGL((k_gemv_float<1, 1, 4>), grid, dim3(256), 0, stream, W, n_out, k, x, rows, y, active);
    else if (vec)
        hipLaunchKernelGGL((k_gemv_float<0, 1, 4>), grid, dim3(256), 0, stream, W, n_out, k, x, rows, y, active);
    else if (bf)
        hipLaunchKernelGGL((k_gemv_float<1, 0, 4>), grid, dim3(256), 0, stream, W, n_out, k, x, rows, y, active);
    else
        hipLaunchKernelGGL((k_gemv_float<0, 0, 4>), grid, dim3(256), 0, stream, W, n_out, k, x, rows, y, active);
}

// GateUpAct{Silu}: y[r][i] = silu(y2[r][i]) * y2[r][n + i], y2 the Gemv of the stacked
// [gate; up] weight (crates/kernels/src/reference/linear.rs:75-112 with the quantized dots of
// the MoE FFN, crates/kernels-cpu/src/moe.rs:529-551: software-exp silu, the product rounded
// once).  Four outputs per thread.
__global__ __launch_bounds__(256) void k_silu_mul(const float* __restrict__ y2, int rows, int n,
                                                  float* __restrict__ y, const uint32_t* __restrict__ active) {
    rows = active_rows(active, 0, rows);
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t i = i0 + q;
        if (i >= (int64_t)rows * n) return;
        const int64_t r = i / n, c = i - r * n;
        y[i] = ref_silu(y2[r * 2 * n + c]) * y2[r * 2 * n + n + c];
    }
}

void launch_silu_mul(const float* y2, int rows, int n, float* y, hipStream_t stream, const uint32_t* active) {
    const int64_t total = (int64_t)rows * n;
    if (total == 0) return;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((total + 1023) / 1024)), dim3(256), 0, stream, y2, rows, n, y,
                       active);
}

}  // namespace syn
