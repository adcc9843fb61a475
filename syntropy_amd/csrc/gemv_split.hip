// Gemv over Q8_0 and Q4_0 weights in the SPLIT layout (layout.hpp: every block's codes, then
// every block's F16 scale), the layout `repack` produces for those types.
//
// Value: crates/kernels-cpu/src/gemv.rs:539-547 (q32_term: (dw * dx) * s with s the exact I32 sum
// of one 32-value block) folded in ascending block order from +0.0 (gemv/portable.rs:114-190),
// bit for bit.  Activations are Q8_0 rows (act_layout(ACT_Q8_0, rows, k)).
//
// 1 to 8 rows (k_gemv_split): one weight row per wavefront, eight per workgroup.  Each wavefront
// load instruction reads 1 KB of the row's codes, 16 bytes a lane: half a Q8_0 block (the pair
// of lanes adds its two exact halves with a lane swap) or a whole Q4_0 block.  The activation
// rows are staged in LDS once per workgroup.  Each block's term is written to LDS and lane r
// folds activation row r's terms in block order.
//
// 9 or more rows, Q8_0 (k_gemm_q8_split): v_mfma_i32_16x16x32_i8 takes one 32-value block of 16
// tokens (A) against 16 weight rows (B): the exact I32 sums of 256 outputs, which the lane owning
// each output scales and folds (one term per block, in block order).  A wavefront covers 16
// weight rows x 32 tokens.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef unsigned int v4u_s __attribute__((ext_vector_type(4)));
typedef int v4i_s __attribute__((ext_vector_type(4)));

// ---- the repack ---------------------------------------------------------------------------------

// One thread per block: GGUF {f16 d; codes} <-> SPLIT (codes, then scales).
__global__ __launch_bounds__(256) void k_split_repack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                      uint64_t nblocks, int cb, int inverse) {
    const uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= nblocks) return;
    const uint64_t bb = (uint64_t)cb + 2;
    if (!inverse) {
        const uint8_t* s = src + g * bb;
        uint8_t* dc = dst + g * (uint64_t)cb;
        for (int i = 0; i < cb; ++i) dc[i] = s[2 + i];
        dst[(uint64_t)cb * nblocks + 2 * g] = s[0];
        dst[(uint64_t)cb * nblocks + 2 * g + 1] = s[1];
    } else {
        uint8_t* d = dst + g * bb;
        const uint8_t* sc = src + g * (uint64_t)cb;
        for (int i = 0; i < cb; ++i) d[2 + i] = sc[i];
        d[0] = src[(uint64_t)cb * nblocks + 2 * g];
        d[1] = src[(uint64_t)cb * nblocks + 2 * g + 1];
    }
}

void launch_split_repack(int ty, const uint8_t* src, uint8_t* dst, uint64_t bytes, int inverse, hipStream_t stream) {
    const int cb = split_code_bytes(ty);
    const uint64_t nblocks = bytes / (uint64_t)(cb + 2);
    if (nblocks == 0) return;
    hipLaunchKernelGGL(k_split_repack, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, stream, src, dst,
                       nblocks, cb, inverse);
}

// ---- 1 to 8 rows ---------------------------------------------------------------------------------

constexpr int SPLIT_WAVES = 8;
constexpr int SPLIT_UNROLL = 4;  // 16-byte weight loads a lane has in flight
constexpr int SPLIT_STAGE_MAX = 48 * 1024;  // LDS bytes of staged activation rows at most

// LDS of the staged activation rows: codes [R][k], then the F32 scales [R][nb], then (Q4_0) the
// 32-value code sums [R][nb].
SYN_HD inline size_t split_act_lds(int ty, int R, int k) {
    const int nb = k / 32;
    return (size_t)R * k + (size_t)R * nb * 4 * (ty == T_Q4_0 ? 2 : 1);
}
// per wavefront, the terms of one load instruction: [R][64 blocks]
SYN_HD inline size_t split_fold_lds(int R) { return (size_t)SPLIT_WAVES * R * 64 * 4; }

// STAGED: the activation rows are copied to LDS first (when they fit), else read from global.
template <int FMT, int R, int STAGED>
__global__ __launch_bounds__(64 * SPLIT_WAVES) void k_gemv_split(const uint8_t* __restrict__ W, int n_out, int k,
                                                                  const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd,
                                                                  const int32_t* __restrict__ xs, int rows,
                                                                  float* __restrict__ y,
                                                                  const uint32_t* __restrict__ active, int first) {
    rows = active_rows(active, first, rows);
    if (rows == 0) return;  // uniform
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int CB = FMT == T_Q8_0 ? 32 : 16;
    constexpr int BPI = FMT == T_Q8_0 ? 32 : 64;  // blocks per wavefront load instruction
    const int nb = k / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (int)blockIdx.x * SPLIT_WAVES + wave;
    const int8_t* aq = xq;
    const float* ad = xd;
    const int32_t* as = xs;
    size_t fold_off = 0;
    if constexpr (STAGED) {
        int8_t* lq = reinterpret_cast<int8_t*>(lds);
        float* ld = reinterpret_cast<float*>(lds + (size_t)R * k);
        int32_t* ls = reinterpret_cast<int32_t*>(lds + (size_t)R * k + (size_t)R * nb * 4);
        for (int i = threadIdx.x; i < rows * k / 16; i += 64 * SPLIT_WAVES)
            reinterpret_cast<v4u_s*>(lq)[i] = reinterpret_cast<const v4u_s*>(xq)[i];
        for (int i = threadIdx.x; i < rows * nb; i += 64 * SPLIT_WAVES) {
            ld[i] = xd[i];
            if constexpr (FMT == T_Q4_0) ls[i] = xs[i];
        }
        aq = lq;
        ad = ld;
        as = ls;
        fold_off = align_up(split_act_lds(FMT, R, k), 16);
        __syncthreads();
    }
    float* buf = reinterpret_cast<float*>(lds + fold_off) + (size_t)wave * R * 64;
    if (row >= n_out) return;  // uniform per wavefront; no workgroup barrier below
    const uint64_t nblocks = (uint64_t)n_out * nb;
    const uint8_t* codes = W + (uint64_t)row * nb * CB;
    const uint16_t* scales = reinterpret_cast<const uint16_t*>(W + (uint64_t)CB * nblocks) + (uint64_t)row * nb;
    const int pieces = FMT == T_Q8_0 ? 2 * nb : nb;  // 16-byte pieces of the row
    float acc = 0.0f;                                // lane r < rows: activation row r's sum
    for (int g0 = 0; g0 < pieces; g0 += 64 * SPLIT_UNROLL) {
        // SPLIT_UNROLL load instructions in flight before the arithmetic
        v4u_s wv[SPLIT_UNROLL];
        float dwv[SPLIT_UNROLL];
#pragma unroll
        for (int u = 0; u < SPLIT_UNROLL; ++u) {
            const int h = g0 + 64 * u + lane;
            const bool ok = h < pieces;
            wv[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const v4u_s*>(codes + 16 * (uint64_t)h))
                       : v4u_s{0u, 0u, 0u, 0u};
            dwv[u] = ok ? f16_to_f32(scales[FMT == T_Q8_0 ? h >> 1 : h]) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < SPLIT_UNROLL; ++u) {
            const int i0 = g0 + 64 * u;
            if (i0 >= pieces) break;  // uniform
            const int h = i0 + lane;
            const bool ok = h < pieces;
            const v4u_s w = wv[u];
            const int b = FMT == T_Q8_0 ? h >> 1 : h;  // the block
            const int b0 = FMT == T_Q8_0 ? i0 >> 1 : i0;
            const float dw = dwv[u];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (r >= rows) break;  // uniform
                int s;
                if constexpr (FMT == T_Q8_0) {
                    const v4u_s x =
                        ok ? *reinterpret_cast<const v4u_s*>(aq + (size_t)r * k + 16 * h) : v4u_s{0u, 0u, 0u, 0u};
                    s = sdot4(w.x, x.x, sdot4(w.y, x.y, sdot4(w.z, x.z, sdot4(w.w, x.w, 0))));
                    s += __shfl_xor(s, 1);  // the block's other half (exact)
                } else {
                    const v4u_s z4 = {0u, 0u, 0u, 0u};
                    const v4u_s x0 = ok ? *reinterpret_cast<const v4u_s*>(aq + (size_t)r * k + 32 * h) : z4;
                    const v4u_s x1 = ok ? *reinterpret_cast<const v4u_s*>(aq + (size_t)r * k + 32 * h + 16) : z4;
                    const uint32_t m = 0x0F0F0F0Fu;
                    s = sdot4(w.x & m, x0.x, sdot4(w.y & m, x0.y, sdot4(w.z & m, x0.z, sdot4(w.w & m, x0.w, 0))));
                    s = sdot4((w.x >> 4) & m, x1.x,
                              sdot4((w.y >> 4) & m, x1.y, sdot4((w.z >> 4) & m, x1.z, sdot4((w.w >> 4) & m, x1.w, s))));
                    if (ok) s -= 8 * as[r * nb + b];  // (n - 8) codes, exact
                }
                const bool writer = ok && (FMT != T_Q8_0 || (h & 1) == 0);
                if (writer) buf[r * 64 + (b - b0)] = (dw * ad[r * nb + b]) * (float)s;
            }
            wave_lds_sync();
            if (lane < rows) {  // this instruction's blocks, in order, into row `lane`'s sum
                const int nbi = nb - b0 < BPI ? nb - b0 : BPI;
                const float* t = buf + lane * 64;
                for (int j = 0; j < nbi; ++j) acc = acc + t[j];
            }
            wave_lds_sync();
        }
    }
    if (lane < rows) y[(int64_t)lane * n_out + row] = acc;
}

static int split_r(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

template <int FMT>
static void launch_split_fmt(const uint8_t* W, int n_out, int k, const uint8_t* ws, int rows, float* y,
                             hipStream_t stream, const uint32_t* active, int first, int64_t ws_rows) {
    const ActLayout L = act_layout(ACT_Q8_0, (uint64_t)ws_rows, (uint64_t)k);
    const int8_t* xq = reinterpret_cast<const int8_t*>(ws + L.codes) + (int64_t)first * k;
    const float* xd = reinterpret_cast<const float*>(ws + L.d) + (int64_t)first * (k / 32);
    const int32_t* xs = reinterpret_cast<const int32_t*>(ws + L.sums) + (int64_t)first * (k / 32);
    float* yr = y + (int64_t)first * n_out;
    const dim3 grid((unsigned)((n_out + SPLIT_WAVES - 1) / SPLIT_WAVES));
    auto go = [&](auto rt) {
        constexpr int RR = decltype(rt)::value;
        const size_t stage = split_act_lds(FMT, RR, k);
        if (stage <= (size_t)SPLIT_STAGE_MAX) {
            const size_t lds = align_up(stage, 16) + split_fold_lds(RR);
            hipLaunchKernelGGL((k_gemv_split<FMT, RR, 1>), grid, dim3(64 * SPLIT_WAVES), lds, stream, W, n_out, k, xq,
                               xd, xs, rows, yr, active, first);
        } else {
            hipLaunchKernelGGL((k_gemv_split<FMT, RR, 0>), grid, dim3(64 * SPLIT_WAVES), split_fold_lds(RR), stream, W,
                               n_out, k, xq, xd, xs, rows, yr, active, first);
        }
    };
    switch (split_r(rows)) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    default: go(std::integral_constant<int, 8>{}); break;
    }
}

// y[r][o] over a SPLIT matrix from rows quantized to Q8_0 in `ws` (act_layout(ACT_Q8_0, rows, k)),
// eight rows at a time.
void launch_gemv_split(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int rows, float* y,
                       hipStream_t stream, const uint32_t* active) {
    for (int r0 = 0; r0 < rows; r0 += 8) {
        const int nr = rows - r0 < 8 ? rows - r0 : 8;
        if (ty == T_Q8_0)
            launch_split_fmt<T_Q8_0>(W, n_out, k, ws, nr, y, stream, active, r0, rows);
        else
            launch_split_fmt<T_Q4_0>(W, n_out, k, ws, nr, y, stream, active, r0, rows);
    }
}

// ---- 9 or more rows, Q8_0: the int8 matrix cores --------------------------------------------------

constexpr int GQ_TT = 2;  // 16-token groups per wavefront

__global__ __launch_bounds__(256) void k_gemm_q8_split(const uint8_t* __restrict__ W, int n_out, int k,
                                                       const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                       int T, float* __restrict__ y,
                                                       const uint32_t* __restrict__ active) {
    T = active_rows(active, 0, T);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, p = lane >> 4;
    const int row0 = ((int)blockIdx.x * 4 + wave) * 16;
    const int t0 = (int)blockIdx.y * 16 * GQ_TT;
    if (row0 >= n_out || t0 >= T) return;  // uniform per wavefront; no barrier below
    const int nb = k / 32;
    const uint64_t nblocks = (uint64_t)n_out * nb;
    const int wr = row0 + c < n_out ? row0 + c : n_out - 1;  // B column c: weight row (clamped)
    const uint8_t* wcodes = W + (uint64_t)wr * nb * 32 + 8 * p;
    const uint16_t* wsc = reinterpret_cast<const uint16_t*>(W + 32 * nblocks) + (uint64_t)wr * nb;
    const int8_t* xa[GQ_TT];
    const float* xdt[GQ_TT][4];
#pragma unroll
    for (int tt = 0; tt < GQ_TT; ++tt) {
        const int ta = t0 + 16 * tt + c;  // A row c: token (clamped)
        xa[tt] = xq + (int64_t)(ta < T ? ta : T - 1) * k + 8 * p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int to = t0 + 16 * tt + 4 * p + i;  // the lane's output tokens
            xdt[tt][i] = xd + (int64_t)(to < T ? to : T - 1) * nb;
        }
    }
    float acc[GQ_TT][4];
#pragma unroll
    for (int tt = 0; tt < GQ_TT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[tt][i] = 0.0f;
    const v4i_s z = {0, 0, 0, 0};
    // the next block's operands are loaded before this block's arithmetic
    long bw = *reinterpret_cast<const long*>(wcodes);
    uint16_t dws = wsc[0];
    long av[GQ_TT];
#pragma unroll
    for (int tt = 0; tt < GQ_TT; ++tt) av[tt] = *reinterpret_cast<const long*>(xa[tt]);
    for (int b = 0; b < nb; ++b) {
        const long bw_c = bw;
        const uint16_t dws_c = dws;
        long av_c[GQ_TT];
#pragma unroll
        for (int tt = 0; tt < GQ_TT; ++tt) av_c[tt] = av[tt];
        if (b + 1 < nb) {
            bw = *reinterpret_cast<const long*>(wcodes + 32 * (b + 1));
            dws = wsc[b + 1];
#pragma unroll
            for (int tt = 0; tt < GQ_TT; ++tt) av[tt] = *reinterpret_cast<const long*>(xa[tt] + 32 * (b + 1));
        }
        const float dw = f16_to_f32(dws_c);
#pragma unroll
        for (int tt = 0; tt < GQ_TT; ++tt) {
            const v4i_s d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av_c[tt], bw_c, z, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tt][i] = acc[tt][i] + (dw * xdt[tt][i][b]) * (float)d[i];
        }
    }
    if (row0 + c < n_out) {
#pragma unroll
        for (int tt = 0; tt < GQ_TT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int to = t0 + 16 * tt + 4 * p + i;
                if (to < T) y[(int64_t)to * n_out + row0 + c] = acc[tt][i];
            }
    }
}

void launch_gemm_q8_split(const uint8_t* W, int n_out, int k, const uint8_t* ws, int T, float* y,
                          hipStream_t stream, const uint32_t* active) {
    const ActLayout L = act_layout(ACT_Q8_0, (uint64_t)T, (uint64_t)k);
    const dim3 grid((unsigned)((n_out + 63) / 64), (unsigned)((T + 16 * GQ_TT - 1) / (16 * GQ_TT)));
    hipLaunchKernelGGL(k_gemm_q8_split, grid, dim3(256), 0, stream, W, n_out, k,
                       reinterpret_cast<const int8_t*>(ws + L.codes), reinterpret_cast<const float*>(ws + L.d), T, y,
                       active);
}

}  // namespace syn
