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
// rows are staged in LDS once per workgroup; a single F32 row can instead be quantized there by
// every workgroup (the same Q8_0 blocks the quantization kernel writes), under the first weight
// loads, which saves the separate quantization launch.  Each block's term is written to LDS and
// lane r folds activation row r's terms in block order.  At one activation row the workgroup's
// rows are folded together, lane w of the first wavefront adding wavefront w's terms, a chunk of
// 128 blocks at a time: one fold instruction serves every row of the workgroup (a lane-0-only
// fold per wavefront costs as many instructions as all the row's other arithmetic together).
//
// 2 or more rows (k_gemm_q8_splitk up to 16 rows of whole 16-block stages, k_gemm_q8_staged for
// more rows or rows of whole 4-block stages, Q8_0 and Q4_0; else for Q8_0 from 9 rows
// k_gemm_q8_split): v_mfma_i32_16x16x32_i8 takes one 32-value block of 16 weight rows against 16
// tokens: the exact I32 sums of 256 outputs, which are scaled and folded (one term per block, in
// block order).
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
// wavefronts of a workgroup that quantizes its row itself: for Q4_0 sixteen quantize the row half
// as often as eight (4096 x 4096: 5.03 against 5.38 us a call, 8192 x 4096: 6.39 against 7.08,
// 4096 x 14336: 11.9 against 12.7) where the matrix has rows for a workgroup of sixteen on each
// of gfx950's 256 CUs; below that, and for Q8_0, whose rows carry twice the bytes, eight
// (Q8_0 14336 x 4096: 12.75 against 13.75 us, 4096 x 14336: 16.5 against 17.2)
constexpr int FUSE_WAVES = 16;
constexpr int FUSE_WAVES_FEW = 8;
constexpr int GFX950_CUS = 256;
constexpr int SPLIT_UNROLL = 4;  // 16-byte weight loads a lane has in flight
constexpr int SPLIT_STAGE_MAX = 48 * 1024;  // LDS bytes of staged activation rows at most

// LDS of the staged activation rows: codes [R][k], then the F32 scales [R][nb], then (Q4_0) the
// 32-value code sums [R][nb].
SYN_HD inline size_t split_act_lds(int ty, int R, int k) {
    const int nb = k / 32;
    return (size_t)R * k + (size_t)R * nb * 4 * (ty == T_Q4_0 ? 2 : 1);
}
// per wavefront, the terms of one load instruction: [R][64 blocks]
SYN_HD inline size_t split_fold_lds(int R, int waves = SPLIT_WAVES) { return (size_t)waves * R * 64 * 4; }
// one activation row: the terms of FOLD_CHUNK blocks of each of the workgroup's rows, a row's
// F32 words padded to a multiple of four plus four, so that the folding lanes' 16-byte reads
// start in different banks
constexpr int FOLD_CHUNK = 128;
SYN_HD inline int wg_fold_stride(int nb) { return ((nb < FOLD_CHUNK ? nb : FOLD_CHUNK) + 3) / 4 * 4 + 4; }
SYN_HD inline size_t wg_fold_lds(int nb, int waves) { return (size_t)waves * wg_fold_stride(nb) * 4; }

// STAGED 1: the activation rows are copied to LDS first (when they fit), 0: read from global;
// 2 (R = 1): the F32 row xf is quantized to Q8_0 blocks in LDS by the workgroup.
// One activation row: eight wavefronts a SIMD (64 VGPRs at most), two workgroups of sixteen or
// four of eight resident on a CU.
template <int FMT, int R, int STAGED, int WVS = STAGED == 2 ? FUSE_WAVES : SPLIT_WAVES>
__global__ __launch_bounds__(64 * WVS, R == 1 ? 8 : 1) void k_gemv_split(const uint8_t* __restrict__ W, int n_out, int k,
                                                                  const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd,
                                                                  const int32_t* __restrict__ xs, int rows,
                                                                  float* __restrict__ y,
                                                                  const uint32_t* __restrict__ active, int first,
                                                                  const float* __restrict__ xf) {
    static_assert(STAGED != 2 || R == 1, "one row quantized in the workgroup");
    constexpr bool WGF = R == 1;  // the workgroup's rows folded together
    rows = active_rows(active, first, rows);
    if (rows == 0) return;  // uniform
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int CB = FMT == T_Q8_0 ? 32 : 16;
    constexpr int BPI = FMT == T_Q8_0 ? 32 : 64;  // blocks per wavefront load instruction
    const int nb = k / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (int)blockIdx.x * WVS + wave;
    const uint64_t nblocks = (uint64_t)n_out * nb;
    const int rowc = row < n_out ? row : n_out - 1;  // a wavefront past the matrix loads its last row, unused
    const uint8_t* codes = W + (uint64_t)rowc * nb * CB;
    const uint16_t* scales = reinterpret_cast<const uint16_t*>(W + (uint64_t)CB * nblocks) + (uint64_t)rowc * nb;
    const int pieces = FMT == T_Q8_0 ? 2 * nb : nb;  // 16-byte pieces of the row
    // SPLIT_UNROLL load instructions (and their scales) in flight before the arithmetic: the
    // loads are unconditional (pieces past the row re-read its last piece, unused) and the
    // scales stay raw bits until used, so no wait splits the group.  The first group is issued
    // before the activation rows are staged.
    v4u_s wv[SPLIT_UNROLL];
    uint16_t swv[SPLIT_UNROLL];
    auto load_group = [&](int g0) {
#pragma unroll
        for (int u = 0; u < SPLIT_UNROLL; ++u) {
            const int h0 = g0 + 64 * u + lane;
            const int h = h0 < pieces ? h0 : pieces - 1;
            wv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u_s*>(codes + 16 * (uint64_t)h));
            swv[u] = scales[FMT == T_Q8_0 ? h >> 1 : h];
        }
    };
    // STAGED 2: the row's first values are loaded before the weights, so that quantizing them
    // waits for them alone (loads retire in order) while the weight loads fly
    constexpr int XPRE = 16 / WVS > 0 ? 16 / WVS : 1;  // passes of 64 WVS lanes (k <= 4096)
    float4 xv[XPRE];
    if constexpr (STAGED == 2) {
#pragma unroll
        for (int q = 0; q < XPRE; ++q) {
            const int t = (int)threadIdx.x + 64 * WVS * q;
            const int tc = t < nb * 8 ? t : 0;
            xv[q] = reinterpret_cast<const float4*>(xf)[tc];  // block tc / 8, values 4 (tc % 8) ..
        }
        __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the weights'
    }
    load_group(0);
    const int8_t* aq = xq;
    const float* ad = xd;
    const int32_t* as = xs;
    size_t fold_off = 0;
    if constexpr (STAGED == 1) {
        int8_t* lq = reinterpret_cast<int8_t*>(lds);
        float* ld = reinterpret_cast<float*>(lds + (size_t)R * k);
        int32_t* ls = reinterpret_cast<int32_t*>(lds + (size_t)R * k + (size_t)R * nb * 4);
        for (int i = threadIdx.x; i < rows * k / 16; i += 64 * WVS)
            reinterpret_cast<v4u_s*>(lq)[i] = reinterpret_cast<const v4u_s*>(xq)[i];
        for (int i = threadIdx.x; i < rows * nb; i += 64 * WVS) {
            ld[i] = xd[i];
            if constexpr (FMT == T_Q4_0) ls[i] = xs[i];
        }
        aq = lq;
        ad = ld;
        as = ls;
        fold_off = align_up(split_act_lds(FMT, R, k), 16);
        __syncthreads();
    } else if constexpr (STAGED == 2) {
        // q8_0_block_lane over eight lanes a block: the blocks of a pass are whole groups of
        // eight lanes, active or not together
        int8_t* lq = reinterpret_cast<int8_t*>(lds);
        float* ld = reinterpret_cast<float*>(lds + (size_t)k);
        int32_t* ls = reinterpret_cast<int32_t*>(lds + (size_t)k + (size_t)nb * 4);
        // lane t % 8 of block t / 8 (values 4 (t % 8) ..); computed by every lane of the pass, so
        // that the preloaded values are used where they were loaded, written where t is a block's
        auto quant = [&](float4 v, int t) {
            const int blk = t >> 3, sub = t & 7;
            const Q8_0Lane q = q8_0_block_lane(v);
            if (t < nb * 8) {
                reinterpret_cast<uint32_t*>(lq + (size_t)blk * 32)[sub] = q.packed;
                if (sub == 0) {
                    ld[blk] = q.d;
                    if constexpr (FMT == T_Q4_0) ls[blk] = q.sum;
                }
            }
        };
#pragma unroll
        for (int q = 0; q < XPRE; ++q) quant(xv[q], (int)threadIdx.x + 64 * WVS * q);
        for (int t = (int)threadIdx.x + 64 * WVS * XPRE; t < nb * 8; t += 64 * WVS)
            quant(reinterpret_cast<const float4*>(xf)[t], t);
        aq = lq;
        ad = ld;
        as = ls;
        fold_off = align_up(split_act_lds(FMT, R, k), 16);
        lds_barrier();  // the LDS rows whole; the weight loads stay in flight
    }
    float* buf = reinterpret_cast<float*>(lds + fold_off) + (size_t)wave * R * 64;
    // WGF: the terms [wavefront][blocks cb ..], the workgroup's rows folded by the first wavefront;
    // a wavefront past the matrix goes on (it reaches the barriers) over its clamped row, unused
    float* terms = reinterpret_cast<float*>(lds + fold_off);
    const int fst = wg_fold_stride(nb);
    int cb = 0;
    if constexpr (!WGF) {
        if (row >= n_out) return;  // uniform per wavefront; no workgroup barrier below
    }
    float acc = 0.0f;  // lane r < rows: activation row r's sum (WGF: lane w of wavefront 0, row w's)
    for (int g0 = 0; g0 < pieces; g0 += 64 * SPLIT_UNROLL) {
        if (g0) load_group(g0);
#pragma unroll
        for (int u = 0; u < SPLIT_UNROLL; ++u) {
            const int i0 = g0 + 64 * u;
            if (i0 >= pieces) break;  // uniform
            const int h = i0 + lane;
            const bool ok = h < pieces;
            const v4u_s w = ok ? wv[u] : v4u_s{0u, 0u, 0u, 0u};
            const int b = FMT == T_Q8_0 ? h >> 1 : h;  // the block
            const int b0 = FMT == T_Q8_0 ? i0 >> 1 : i0;
            const float dw = ok ? f16_to_f32(swv[u]) : 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (r >= rows) break;  // uniform
                int s;
                if constexpr (FMT == T_Q8_0) {
                    const v4u_s x =
                        ok ? *reinterpret_cast<const v4u_s*>(aq + (size_t)r * k + 16 * h) : v4u_s{0u, 0u, 0u, 0u};
                    s = sdot4(w.x, x.x, sdot4(w.y, x.y, sdot4(w.z, x.z, sdot4(w.w, x.w, 0))));
                    s += __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, false);  // the block's other half (lane ^ 1; exact)
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
                const float term = (dw * ad[r * nb + b]) * (float)s;
                if constexpr (WGF) {
                    if (writer) terms[wave * fst + (b - cb)] = term;
                } else {
                    if (writer) buf[r * 64 + (b - b0)] = term;
                }
            }
            if constexpr (WGF) {
                const int done = nb - b0 < BPI ? nb : b0 + BPI;  // blocks through this instruction
                if (done - cb == FOLD_CHUNK || done == nb) {      // uniform
                    lds_barrier();
                    if (wave == 0 && lane < WVS) {  // blocks cb .. done - 1 of row `lane`, in order
                        const float* t = terms + lane * fst;
                        const int cnt = done - cb;
                        int j = 0;
                        for (; j + 32 <= cnt; j += 32) {  // eight reads in flight
                            float4 v[8];
#pragma unroll
                            for (int q = 0; q < 8; ++q) v[q] = reinterpret_cast<const float4*>(t + j)[q];
#pragma unroll
                            for (int q = 0; q < 8; ++q) acc = (((acc + v[q].x) + v[q].y) + v[q].z) + v[q].w;
                        }
                        for (; j < cnt; ++j) acc = acc + t[j];
                    }
                    cb = done;
                    if (done < nb) lds_barrier();  // read out before the next chunk's terms
                }
            } else {
                wave_lds_sync();
                if (lane < rows) {  // this instruction's blocks, in order, into row `lane`'s sum
                    const int nbi = nb - b0 < BPI ? nb - b0 : BPI;
                    const float* t = buf + lane * 64;
                    for (int j = 0; j < nbi; ++j) acc = acc + t[j];
                }
                wave_lds_sync();
            }
        }
    }
    if constexpr (WGF) {
        const int orow = (int)blockIdx.x * WVS + lane;
        if (wave == 0 && lane < WVS && orow < n_out) y[orow] = acc;
    } else if (lane < rows) {
        y[(int64_t)lane * n_out + row] = acc;
    }
}

static int split_r(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

// Whether one launch of `rows` <= 8 rows stages its activation rows in LDS.
bool gemv_split_staged(int ty, int rows, int k) {
    return split_act_lds(ty, split_r(rows), k) <= (size_t)SPLIT_STAGE_MAX;
}

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
        const size_t fold = RR == 1 ? wg_fold_lds(k / 32, SPLIT_WAVES) : split_fold_lds(RR);
        if (stage <= (size_t)SPLIT_STAGE_MAX) {
            const size_t lds = align_up(stage, 16) + fold;
            hipLaunchKernelGGL((k_gemv_split<FMT, RR, 1>), grid, dim3(64 * SPLIT_WAVES), lds, stream, W, n_out, k, xq,
                               xd, xs, rows, yr, active, first, nullptr);
        } else {
            hipLaunchKernelGGL((k_gemv_split<FMT, RR, 0>), grid, dim3(64 * SPLIT_WAVES), fold, stream, W,
                               n_out, k, xq, xd, xs, rows, yr, active, first, nullptr);
        }
    };
    switch (split_r(rows)) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    default: go(std::integral_constant<int, 8>{}); break;
    }
}

// One F32 row quantized inside the product's workgroups (no workspace): where its Q8_0 blocks fit
// the LDS staging area.
bool gemv_split_fused_fits(int ty, int k) { return split_act_lds(ty, 1, k) <= (size_t)SPLIT_STAGE_MAX; }

void launch_gemv_split_fused(int ty, const uint8_t* W, int n_out, int k, const float* x, float* y, hipStream_t stream,
                             const uint32_t* active) {
    auto go = [&](auto wt) {
        constexpr int WV = decltype(wt)::value;
        const dim3 grid((unsigned)((n_out + WV - 1) / WV));
        const size_t lds = align_up(split_act_lds(ty, 1, k), 16) + wg_fold_lds(k / 32, WV);
        if (ty == T_Q8_0)
            hipLaunchKernelGGL((k_gemv_split<T_Q8_0, 1, 2, WV>), grid, dim3(64 * WV), lds, stream, W, n_out, k,
                               nullptr, nullptr, nullptr, 1, y, active, 0, x);
        else
            hipLaunchKernelGGL((k_gemv_split<T_Q4_0, 1, 2, WV>), grid, dim3(64 * WV), lds, stream, W, n_out, k,
                               nullptr, nullptr, nullptr, 1, y, active, 0, x);
    };
    if (ty == T_Q4_0 && n_out >= FUSE_WAVES * GFX950_CUS)
        go(std::integral_constant<int, FUSE_WAVES>{});
    else
        go(std::integral_constant<int, FUSE_WAVES_FEW>{});
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
//
// A wavefront owns 16 weight rows x 16 TT tokens.  Per block, v_mfma_i32_16x16x32_i8 takes the
// rows' codes as A (lane c: row c's 8 codes at 8 p of the block, p = lane / 16) and the tokens'
// codes as B (lane c: token c's codes at 8 p): lane (c, p) receives the exact sums of rows 4 p + i
// against token c, scales them by (dw * dx) and adds them to its accumulators in block order.
// Loads come in groups of four blocks, the next group's issued before the current one's
// arithmetic; with whole pairs of groups (nb % 8 == 0) a lane reads a row's four scales and a
// token's four activation scales with one load each.  The workgroup's wavefronts share the 16 rows and take
// consecutive token tiles, so the rows' codes are fetched once into the caches.

constexpr int GQ_G = 4;  // blocks per load group

template <int TT>
struct GqGroup {
    long w[GQ_G];        // row c's codes, 8 bytes of each block
    uint32_t sc[4][2];   // rows 4 p + i: four F16 scales
    long a[TT][GQ_G];    // token c of tile tt: 8 codes of each block
    float dx[TT][GQ_G];  // token c of tile tt: each block's scale
};

template <int TT, bool VEC>
__device__ __forceinline__ void gq_load(GqGroup<TT>& g, const uint8_t* wrow, const uint16_t* const* srow,
                                        const int8_t* const* xa, const float* const* xdt, int b0, int nb) {
    if constexpr (VEC) {  // a whole group, 8- and 16-byte aligned
#pragma unroll
        for (int j = 0; j < GQ_G; ++j) g.w[j] = *reinterpret_cast<const long*>(wrow + 32 * (b0 + j));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint2 v = *reinterpret_cast<const uint2*>(srow[i] + b0);
            g.sc[i][0] = v.x;
            g.sc[i][1] = v.y;
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int j = 0; j < GQ_G; ++j) g.a[t][j] = *reinterpret_cast<const long*>(xa[t] + 32 * (b0 + j));
            const float4 d = *reinterpret_cast<const float4*>(xdt[t] + b0);
            g.dx[t][0] = d.x;
            g.dx[t][1] = d.y;
            g.dx[t][2] = d.z;
            g.dx[t][3] = d.w;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < GQ_G; ++j) {
        const bool ok = b0 + j < nb;
        g.w[j] = ok ? *reinterpret_cast<const long*>(wrow + 32 * (b0 + j)) : 0;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            g.a[t][j] = ok ? *reinterpret_cast<const long*>(xa[t] + 32 * (b0 + j)) : 0;
            g.dx[t][j] = ok ? xdt[t][b0 + j] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t h[GQ_G];
#pragma unroll
        for (int j = 0; j < GQ_G; ++j) h[j] = b0 + j < nb ? srow[i][b0 + j] : 0u;
        g.sc[i][0] = h[0] | (h[1] << 16);
        g.sc[i][1] = h[2] | (h[3] << 16);
    }
}

// The arithmetic of one group: the group's MFMAs first, then each block's terms in block order.
template <int TT, bool VEC>
__device__ __forceinline__ void gq_compute(const GqGroup<TT>& g, float (&acc)[TT][4], int b0, int nb) {
    const v4i_s z = {0, 0, 0, 0};
    v4i_s d[GQ_G][TT];
#pragma unroll
    for (int j = 0; j < GQ_G; ++j)
#pragma unroll
        for (int t = 0; t < TT; ++t) d[j][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(g.w[j], g.a[t][j], z, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < GQ_G; ++j) {
        if (!VEC && b0 + j >= nb) break;  // uniform
        float dw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[i] = f16_to_f32((uint16_t)(g.sc[i][j >> 1] >> (16 * (j & 1))));
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = acc[t][i] + (dw[i] * g.dx[t][j]) * (float)d[j][t][i];
    }
}

template <int TT, bool VEC>
__global__ __launch_bounds__(256) void k_gemm_q8_split(const uint8_t* __restrict__ W, int n_out, int k,
                                                       const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                       int T, float* __restrict__ y,
                                                       const uint32_t* __restrict__ active) {
    T = active_rows(active, 0, T);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, p = lane >> 4;
    const int row0 = (int)blockIdx.x * 16;
    const int t0 = ((int)blockIdx.y * (int)(blockDim.x >> 6) + wave) * 16 * TT;
    if (t0 >= T) return;  // uniform per wavefront; no barrier below
    const int nb = k / 32;
    const uint64_t nblocks = (uint64_t)n_out * nb;
    const int wr = row0 + c < n_out ? row0 + c : n_out - 1;  // A row c: weight row (clamped)
    const uint8_t* wrow = W + (uint64_t)wr * nb * 32 + 8 * p;
    const uint16_t* scales = reinterpret_cast<const uint16_t*>(W + 32 * nblocks);
    const uint16_t* srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = row0 + 4 * p + i;  // the lane's output rows (clamped)
        srow[i] = scales + (uint64_t)(r < n_out ? r : n_out - 1) * nb;
    }
    const int8_t* xa[TT];
    const float* xdt[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tok = t0 + 16 * t + c;  // B column c: token (clamped)
        const int tc = tok < T ? tok : T - 1;
        xa[t] = xq + (int64_t)tc * k + 8 * p;
        xdt[t] = xd + (int64_t)tc * nb;
    }
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = 0.0f;
    // two groups in registers, each loaded while the other one's arithmetic runs.  The loads are
    // unconditional (a group past the row reloads the current one), so that the wait before each
    // group's arithmetic counts only the other group's loads.
    // With VEC the row holds whole pairs of groups (nb % 8 == 0) and nothing is conditional.
    GqGroup<TT> ga, gb;
    gq_load<TT, VEC>(ga, wrow, srow, xa, xdt, 0, nb);
    for (int b0 = 0; b0 < nb; b0 += 2 * GQ_G) {
        const bool second = VEC || b0 + GQ_G < nb;
        gq_load<TT, VEC>(gb, wrow, srow, xa, xdt, second ? b0 + GQ_G : b0, nb);
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the arithmetic
        gq_compute<TT, VEC>(ga, acc, b0, nb);
        __builtin_amdgcn_sched_barrier(0);
        gq_load<TT, VEC>(ga, wrow, srow, xa, xdt, b0 + 2 * GQ_G < nb ? b0 + 2 * GQ_G : b0, nb);
        __builtin_amdgcn_sched_barrier(0);
        if (second) gq_compute<TT, VEC>(gb, acc, b0 + GQ_G, nb);
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tok = t0 + 16 * t + c;
        if (tok >= T) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = row0 + 4 * p + i;
            if (r < n_out) y[(int64_t)tok * n_out + r] = acc[t][i];
        }
    }
}

// ---- the staged GEMM: weights, codes and scales streamed into an LDS ring -------------------------
//
// A workgroup takes 32 weight rows (two wavefront row groups of 16) x TW = 16 TT TG tokens (TG
// token groups of 16 TT), stage by stage: four blocks of every operand are copied into LDS by
// global_load_lds while earlier stages compute.  Stage layout (bytes), WL = 4 CB (the rows' code
// bytes per stage: 128 for Q8_0, 64 for Q4_0):
//   codes of the rows   [row][WL]       32 WL  a row's four blocks, swizzled (below)
//   codes of the tokens [token][128]    128 TW the same as Q8_0 rows
//   row scales          [row][block] F16  256
//   token scales        [token][block] F32 16 TW
// A copy instruction moves 1 KB, 16 bytes a lane: eight 128-byte lines (Q8_0 rows, tokens) or
// sixteen 64-byte Q4_0 row lines.  Within a 128-byte line the 16-byte halves of the four blocks
// are stored at slot 2 (j ^ ((c >> 1) & 3)) + (h ^ (c >> 3)) for block j, half h of the line's
// row or token c (mod 16); within a 64-byte Q4_0 line block j sits at slot j ^ ((c >> 2) & 3).
// Either way a matrix operand read (16 lines, 8 bytes of each for each of two lane quarters per
// half-wavefront) covers 256 distinct bytes modulo 256: every bank once.
// A wavefront issues the same number of copies every stage, so its wait is a fixed count.
//
// Q4_0: lane (c, p) takes the low nibbles (p < 2) or the high nibbles (p >= 2) of bytes 8 (p & 1)
// .. +7 of the block's 16: elements 8 p .. 8 p + 7 of the block, the same elements as the token
// operand's 8 bytes at 8 p.  The nibbles n become the int8 values n - 8 per byte with
// ((n + 0x78) ^ 0x80), which no byte carries out of, so the sums are the block's exact
// sum of (n - 8) x.

constexpr int QS_S = 4;    // blocks per stage
constexpr int QS_RW = 32;  // weight rows per workgroup
constexpr int QS_NS_MAX = 3;

template <int FMT, int TT, int TG>
struct QsCfg {
    static constexpr int CB = FMT == T_Q8_0 ? 32 : 16;  // code bytes per block
    static constexpr int WL = QS_S * CB;                 // a row's code bytes per stage
    static constexpr int NW = 2 * TG;                    // wavefronts
    static constexpr int TW = 16 * TT * TG;              // tokens
    static constexpr int W_OFF = 0, A_OFF = QS_RW * WL;
    static constexpr int SC_OFF = A_OFF + TW * QS_S * 32;
    static constexpr int DX_OFF = SC_OFF + QS_RW * QS_S * 2;
    static constexpr int STAGE = DX_OFF + TW * QS_S * 4;
    // stages a barrier step consumes: two for one token tile a wavefront pair (few tokens), else one
    static constexpr int SPI = TT == 1 && TG == 1 ? 2 : 1;
    // ring stages: as many as 64 KB hold, at most QS_NS_MAX (three stages a step beyond one)
    static constexpr int NSM = SPI == 2 ? 6 : QS_NS_MAX;
    static constexpr int NS = 64 * 1024 / STAGE < NSM ? 64 * 1024 / STAGE : NSM;
    // copies per stage: row codes, token codes, and the two scale sets, each set whole or in
    // SPARTS / DPARTS parts, so that the count splits evenly over the wavefronts
    static constexpr int WCOPIES = QS_RW * WL / 1024;
    static constexpr int SPARTS = TG == 1 || (FMT == T_Q4_0 && TG == 2) ? 1 : 2;
    static constexpr int DPARTS = TG == 1 ? 1 : FMT == T_Q8_0 ? 2 : TG == 4 ? 4 : 1;
    static constexpr int TOTAL = WCOPIES + TW / 8 + SPARTS + DPARTS;
    static constexpr int COPIES = TOTAL / NW;  // per wavefront per stage
    static_assert(TOTAL % NW == 0, "copies split evenly");
    static_assert(NS >= 2 * SPI && COPIES * (NS - 2 * SPI) <= 63, "the wait count fits vmcnt");
};

// The LDS byte offset, within its 128-byte line, of block j's 8 bytes at 8 p for line c.
SYN_DEV int qs_slot(int c, int j, int p) {
    return 32 * (j ^ ((c >> 1) & 3)) + 16 * ((p >> 1) ^ ((c >> 3) & 1)) + 8 * (p & 1);
}
// The same within a 64-byte Q4_0 row line: block j's 8 bytes at 8 (p & 1).
SYN_DEV int qs_slot4(int c, int j, int p) { return 16 * (j ^ ((c >> 2) & 3)) + 8 * (p & 1); }

// RN(h * x) for the F16 half `hi` of word w and an F32 x: v_fma_mix_f32 converts the half inside
// the instruction (exactly) and adds +0.0, which rounds the product once; only a zero product's
// sign can differ from a multiply (+0.0 for -0.0), which a sum that starts from +0.0 does not see.
SYN_DEV float f16_mul_f32(uint32_t w, int hi, float x) {
    float p;
    if (hi)
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(p) : "v"(w), "v"(x));
    else
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(p) : "v"(w), "v"(x));
    return p;
}

// Four Q4_0 code bytes -> the int8 values n - 8 of their low (sh 0) or high (sh 4) nibbles.
SYN_DEV uint32_t q4_signed(uint32_t v, int sh) {
    return (((v >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

// The lane's part of its wavefront's copies: per copy a global base (advanced per stage by
// `step` bytes), the lane's 32-bit offset, the LDS offset in the stage, 16 or 4 bytes, and whether
// the lane takes part.
struct QsCopy {
    const uint8_t* base;
    uint32_t voff, lds, step;
    bool wide, on;
};

template <int FMT, int TT, int TG>
__device__ __forceinline__ void qs_plan(QsCopy* cp, const uint8_t* W, const uint8_t* scales, const int8_t* xq,
                                        const float* xd, int n_out, int nb, int k, int T, int row0, int t0, int wave,
                                        int lane) {
    using C = QsCfg<FMT, TT, TG>;
    const uint32_t rb = (uint32_t)nb * (uint32_t)C::CB;
    auto wrow = [&](int r) { return (uint32_t)(row0 + r < n_out ? row0 + r : n_out - 1); };
    auto tok = [&](int t) { return (uint32_t)(t0 + t < T ? t0 + t : T - 1); };
    // lane -> line 8 q + lane / 8 of the stage, LDS slot lane % 8, holding the line's bytes at
    // `src` (the inverse of the swizzle)
    const int slot = lane & 7, li = lane >> 3;
    auto src = [&](int c) {
        const int j = (slot >> 1) ^ ((c >> 1) & 3), h = (slot & 1) ^ ((c >> 3) & 1);
        return (uint32_t)(32 * j + 16 * h);
    };
    auto wcopy = [&](int q) {
        if constexpr (FMT == T_Q8_0) {
            const int r = 8 * q + li;
            return QsCopy{W, wrow(r) * rb + src(r & 15), (uint32_t)(C::W_OFF + 1024 * q), (uint32_t)C::WL, true, true};
        } else {  // lane -> row 16 q + lane / 4, slot lane % 4 holding block (lane % 4) ^ ((row >> 2) & 3)
            const int r = 16 * q + (lane >> 2);
            return QsCopy{W, wrow(r) * rb + 16u * (uint32_t)((lane & 3) ^ ((r >> 2) & 3)),
                          (uint32_t)(C::W_OFF + 1024 * q), (uint32_t)C::WL, true, true};
        }
    };
    auto acopy = [&](int q) {
        const int t = 8 * q + li;
        return QsCopy{reinterpret_cast<const uint8_t*>(xq), tok(t) * (uint32_t)k + src(t & 15),
                      (uint32_t)(C::A_OFF + 1024 * q), 32u * QS_S, true, true};
    };
    // part h of `parts` of the row scales (32 rows x 8 bytes): lane -> row (32 / parts) h + lane / 2,
    // blocks 2 (lane % 2), +1, from the lanes below 64 / parts
    auto scopy = [&](int h, int parts) {
        const int r = (32 / parts) * h + (lane >> 1);
        return QsCopy{scales, wrow(r) * (uint32_t)nb * 2u + 4u * (uint32_t)(lane & 1),
                      (uint32_t)(C::SC_OFF + (256 / parts) * h), 2u * QS_S, false, lane < 64 / parts};
    };
    // part h of `parts` of the token scales (TW <= 64 tokens x 16 bytes): lane -> token
    // (TW / parts) h + lane, from the lanes below TW / parts
    auto dcopy = [&](int h, int parts) {
        const int t = (C::TW / parts) * h + lane;
        return QsCopy{reinterpret_cast<const uint8_t*>(xd), tok(t) * (uint32_t)nb * 4u,
                      (uint32_t)(C::DX_OFF + 16 * (C::TW / parts) * h), 4u * QS_S, true, lane < C::TW / parts};
    };
    constexpr int S = C::SPARTS, D = C::DPARTS;
    if constexpr (FMT == T_Q8_0 && TT == 1 && TG == 1) {  // 8 copies: 4 row, 2 token, two scale sets
        cp[0] = wcopy(2 * wave);
        cp[1] = wcopy(2 * wave + 1);
        cp[2] = acopy(wave);
        cp[3] = wave == 0 ? scopy(0, S) : dcopy(0, D);
    } else if constexpr (FMT == T_Q8_0 && TG == 1) {  // 10 copies: 4 row, 4 token, two scale sets
        cp[0] = wcopy(2 * wave);
        cp[1] = wcopy(2 * wave + 1);
        cp[2] = acopy(2 * wave);
        cp[3] = acopy(2 * wave + 1);
        cp[4] = wave == 0 ? scopy(0, S) : dcopy(0, D);
    } else if constexpr (FMT == T_Q8_0 && TT == 2) {  // 16 copies: 4 row, 8 token, halves of the scale sets
        cp[0] = wcopy(wave);
        cp[1] = acopy(2 * wave);
        cp[2] = acopy(2 * wave + 1);
        cp[3] = wave < 2 ? scopy(wave, S) : dcopy(wave - 2, D);
    } else if constexpr (FMT == T_Q8_0 && TG == 2) {  // 12 copies: 4 row, 4 token, halves of the scale sets
        cp[0] = wcopy(wave);
        cp[1] = acopy(wave);
        cp[2] = wave < 2 ? scopy(wave, S) : dcopy(wave - 2, D);
    } else if constexpr (FMT == T_Q8_0) {  // TG 4, 16 copies: 4 row, 8 token, halves of the scale sets
        cp[0] = acopy(wave);
        cp[1] = wave < 4 ? wcopy(wave) : wave < 6 ? scopy(wave - 4, S) : dcopy(wave - 6, D);
    } else if constexpr (TT == 1 && TG == 1) {  // Q4_0, 6 copies: 2 row, 2 token, two scale sets
        cp[0] = wcopy(wave);
        cp[1] = acopy(wave);
        cp[2] = wave == 0 ? scopy(0, S) : dcopy(0, D);
    } else if constexpr (TG == 1) {  // Q4_0, 8 copies: 2 row, 4 token, two scale sets
        cp[0] = wcopy(wave);
        cp[1] = acopy(2 * wave);
        cp[2] = acopy(2 * wave + 1);
        cp[3] = wave == 0 ? scopy(0, S) : dcopy(0, D);
    } else if constexpr (TT == 2) {  // Q4_0, 12 copies: 2 row, 8 token, two scale sets
        cp[0] = acopy(2 * wave);
        cp[1] = acopy(2 * wave + 1);
        cp[2] = wave < 2 ? wcopy(wave) : wave == 2 ? scopy(0, S) : dcopy(0, D);
    } else if constexpr (TG == 2) {  // Q4_0, 8 copies: 2 row, 4 token, two scale sets
        cp[0] = acopy(wave);
        cp[1] = wave < 2 ? wcopy(wave) : wave == 2 ? scopy(0, S) : dcopy(0, D);
    } else {  // Q4_0, TG 4, 16 copies: 2 row, 8 token, scale halves, token-scale quarters
        cp[0] = acopy(wave);
        cp[1] = wave < 2 ? wcopy(wave) : wave < 4 ? scopy(wave - 2, S) : dcopy(wave - 4, D);
    }
}

template <int FMT, int TT, int TG>
__device__ __forceinline__ void qs_issue(const QsCopy* cp, uint32_t stage_lds, int s) {
#pragma unroll
    for (int u = 0; u < QsCfg<FMT, TT, TG>::COPIES; ++u) {
        const uint8_t* base = cp[u].base + (size_t)cp[u].step * (size_t)s;
        if (cp[u].on) {
            if (cp[u].wide)
                lds_dma16(cp[u].voff, base, stage_lds + cp[u].lds);
            else
                lds_dma4(cp[u].voff, base, stage_lds + cp[u].lds);
        }
    }
}

template <int FMT, int TT, int TG>
__global__ __launch_bounds__(64 * 2 * TG) void k_gemm_q8_staged(const uint8_t* __restrict__ W, int n_out, int k,
                                                                 const int8_t* __restrict__ xq,
                                                                 const float* __restrict__ xd, int T,
                                                                 float* __restrict__ y,
                                                                 const uint32_t* __restrict__ active) {
    using C = QsCfg<FMT, TT, TG>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    T = active_rows(active, 0, T);
    const int row0 = (int)blockIdx.x * QS_RW, t0 = (int)blockIdx.y * C::TW;
    if (t0 >= T) return;  // uniform per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: copy bases in SGPRs
    const int c = lane & 15, p = lane >> 4;
    const int rg = wave & 1, tg = wave >> 1;  // the wavefront's row group and token group
    const int nb = k / 32, nst = nb / QS_S;
    const uint8_t* scales = W + (uint64_t)C::CB * (uint64_t)n_out * (uint64_t)nb;
    QsCopy cp[C::COPIES];
    qs_plan<FMT, TT, TG>(cp, W, scales, xq, xd, n_out, nb, k, T, row0, t0, wave, lane);
    const uint32_t ring = lds_addr(lds);
#pragma unroll
    for (int s = 0; s < C::NS - C::SPI; ++s)
        qs_issue<FMT, TT, TG>(cp, ring + (uint32_t)(C::STAGE * s), s < nst ? s : nst - 1);
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = 0.0f;
    const v4i_s z = {0, 0, 0, 0};
    auto body = [&](int s) __attribute__((always_inline)) {
        const uint8_t* st = lds + C::STAGE * (s % C::NS);
        // the lane's rows 4 p + i: four scales each, 8 bytes a row
        const v4u_s sc01 = *reinterpret_cast<const v4u_s*>(st + C::SC_OFF + (16 * rg + 4 * p) * 8);
        const v4u_s sc23 = *reinterpret_cast<const v4u_s*>(st + C::SC_OFF + (16 * rg + 4 * p) * 8 + 16);
        const uint32_t scw[4][2] = {{sc01.x, sc01.y}, {sc01.z, sc01.w}, {sc23.x, sc23.y}, {sc23.z, sc23.w}};
        float dx[TT][QS_S];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const float4 v = *reinterpret_cast<const float4*>(st + C::DX_OFF + (16 * TT * tg + 16 * t + c) * 16);
            dx[t][0] = v.x;
            dx[t][1] = v.y;
            dx[t][2] = v.z;
            dx[t][3] = v.w;
        }
        v4i_s d[QS_S][TT];
#pragma unroll
        for (int j = 0; j < QS_S; ++j) {
            const int o = qs_slot(c, j, p);  // line c's (row or token, mod 16) bytes 8 p of block j
            long a;
            if constexpr (FMT == T_Q8_0) {
                a = *reinterpret_cast<const long*>(st + C::W_OFF + (16 * rg + c) * C::WL + o);
            } else {
                const uint2 v = *reinterpret_cast<const uint2*>(st + C::W_OFF + (16 * rg + c) * C::WL + qs_slot4(c, j, p));
                const int sh = 4 * (p >> 1);
                a = (long)(((uint64_t)q4_signed(v.y, sh) << 32) | (uint64_t)q4_signed(v.x, sh));
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const long b = *reinterpret_cast<const long*>(st + C::A_OFF + (16 * TT * tg + 16 * t + c) * 128 + o);
                d[j][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < QS_S; ++j) {
            if constexpr (TT == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[0][i] = acc[0][i] + f16_mul_f32(scw[i][j >> 1], j & 1, dx[0][j]) * (float)d[j][0][i];
            } else {
                float dw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) dw[i] = f16_to_f32((uint16_t)(scw[i][j >> 1] >> (16 * (j & 1))));
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][i] = acc[t][i] + (dw[i] * dx[t][j]) * (float)d[j][t][i];
            }
        }
    };
    // SPI stages a barrier: their copies have landed (the NS - 2 SPI after them may fly), the
    // previous step's are read out, and the next SPI go into those slots
    for (int s = 0; s < nst; s += C::SPI) {
        wait_vm<C::COPIES * (C::NS - 2 * C::SPI)>();
        lds_barrier();
#pragma unroll
        for (int u = 0; u < C::SPI; ++u) {
            const int sn = s + C::NS - C::SPI + u;
            qs_issue<FMT, TT, TG>(cp, ring + (uint32_t)(C::STAGE * (sn % C::NS)), sn < nst ? sn : nst - 1);
        }
#pragma unroll
        for (int u = 0; u < C::SPI; ++u)
            if (s + u < nst) body(s + u);  // uniform
    }
    wait_vm<0>();  // the last (repeated) copies have landed before the workgroup ends
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tk = t0 + 16 * TT * tg + 16 * t + c;
        if (tk >= T) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = row0 + 16 * rg + 4 * p + i;
            if (r < n_out) y[(int64_t)tk * n_out + r] = acc[t][i];
        }
    }
}

// ---- up to 16 rows: the K-split staged GEMM ------------------------------------------------------
//
// A workgroup of four wavefronts owns one 16-row x 16-token tile.  A stage holds 16 blocks of
// every operand; wavefront w takes blocks 4w .. 4w + 3 of it, as a slice laid out like a stage of
// k_gemm_q8_staged (the same lines and swizzles), computes the terms (dw dx) s of its blocks for
// the tile's 256 outputs and writes them to LDS.  After the next barrier lane o of the workgroup
// adds output o's 16 terms of the stage to its sum, in block order: the fold, and every bit, is
// the one-wavefront kernel's, with four wavefronts on the tile and a quarter of the stages each.
// Terms of output o sit at [o][16 blocks], wavefront w's four at 16-byte slot w ^ (o & 3).
constexpr int QK_SLICES = 4;             // wavefronts, one 4-block slice of a stage each
constexpr int QK_SB = QS_S * QK_SLICES;  // blocks per stage
constexpr int QK_NS = 2;                 // ring stages

template <int FMT>
struct QkCfg {
    static constexpr int CB = FMT == T_Q8_0 ? 32 : 16;
    static constexpr int WL = QS_S * CB;                        // a row's bytes in a slice
    static constexpr int W_OFF = 0;                             // [slice][16 rows][WL]
    static constexpr int A_OFF = QK_SLICES * 16 * WL;           // [slice][16 tokens][128]
    static constexpr int SC_OFF = A_OFF + QK_SLICES * 16 * 128;  // [16 rows][16 blocks] F16
    static constexpr int DX_OFF = SC_OFF + 16 * QK_SB * 2;       // [16 tokens][16 blocks] F32
    static constexpr int STAGE = DX_OFF + 16 * QK_SB * 4;
    static constexpr int TERMS = 256 * QK_SB * 4;               // [256 outputs][16 blocks] F32
    static constexpr int LDS = QK_NS * STAGE + 2 * TERMS;
    static constexpr int WCOP = 16 * WL / 1024;  // row-line copies of a slice: 2 (Q8_0) or 1 (Q4_0)
    static constexpr int COP = WCOP + 2 + 1;     // + 2 token-line copies + a scale copy (wavefronts 0, 1)
};

template <int FMT>
__global__ __launch_bounds__(256) void k_gemm_q8_splitk(const uint8_t* __restrict__ W, int n_out, int k,
                                                         const int8_t* __restrict__ xq,
                                                         const float* __restrict__ xd, int T,
                                                         float* __restrict__ y,
                                                         const uint32_t* __restrict__ active) {
    using C = QkCfg<FMT>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    T = active_rows(active, 0, T);
    const int row0 = (int)blockIdx.x * 16, t0 = (int)blockIdx.y * 16;
    if (t0 >= T) return;  // uniform per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: copy bases in SGPRs
    const int c = lane & 15, p = lane >> 4;
    const int nb = k / 32, nst = nb / QK_SB;
    const uint32_t rb = (uint32_t)nb * (uint32_t)C::CB;
    const uint8_t* scales = W + (uint64_t)C::CB * (uint64_t)n_out * (uint64_t)nb;
    auto wrow = [&](int r) { return (uint32_t)(row0 + r < n_out ? row0 + r : n_out - 1); };
    auto tok = [&](int t) { return (uint32_t)(t0 + t < T ? t0 + t : T - 1); };
    // this wavefront's copies: its slice's row and token lines, and for wavefronts 0 and 1 the
    // stage's row scales (32 bytes a row) or token scales (64 bytes a token)
    QsCopy cp[C::COP];
    const int slot = lane & 7, li = lane >> 3;
    auto src128 = [&](int cc) {  // the inverse of the 128-byte line swizzle (qs_slot)
        const int j = (slot >> 1) ^ ((cc >> 1) & 3), h = (slot & 1) ^ ((cc >> 3) & 1);
        return (uint32_t)(32 * j + 16 * h);
    };
    const uint32_t wslice = (uint32_t)(4 * wave) * (uint32_t)C::CB;  // the slice's first block in a row
    int ncop = 0;
#pragma unroll
    for (int q = 0; q < C::WCOP; ++q) {
        if constexpr (FMT == T_Q8_0) {
            const int r = 8 * q + li;
            cp[ncop++] = QsCopy{W, wrow(r) * rb + wslice + src128(r), (uint32_t)(C::W_OFF + wave * 16 * C::WL + 1024 * q),
                                (uint32_t)(QK_SB * C::CB), true, true};
        } else {
            const int r = lane >> 2;
            cp[ncop++] = QsCopy{W, wrow(r) * rb + wslice + 16u * (uint32_t)((lane & 3) ^ ((r >> 2) & 3)),
                                (uint32_t)(C::W_OFF + wave * 16 * C::WL), (uint32_t)(QK_SB * C::CB), true, true};
        }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int t = 8 * q + li;
        cp[ncop++] = QsCopy{reinterpret_cast<const uint8_t*>(xq), tok(t) * (uint32_t)k + (uint32_t)(4 * wave * 32) + src128(t),
                            (uint32_t)(C::A_OFF + wave * 2048 + 1024 * q), (uint32_t)(QK_SB * 32), true, true};
    }
    if (wave == 0)
        cp[ncop++] = QsCopy{scales, wrow(lane >> 1) * (uint32_t)nb * 2u + 16u * (uint32_t)(lane & 1),
                            (uint32_t)C::SC_OFF, (uint32_t)(QK_SB * 2), true, lane < 32};
    else if (wave == 1)
        cp[ncop++] = QsCopy{reinterpret_cast<const uint8_t*>(xd), tok(lane >> 2) * (uint32_t)nb * 4u + 16u * (uint32_t)(lane & 3),
                            (uint32_t)C::DX_OFF, (uint32_t)(QK_SB * 4), true, true};
    const uint32_t ring = lds_addr(lds);
    auto issue = [&](int s) {
        const uint32_t st = ring + (uint32_t)(C::STAGE * (s % QK_NS));
#pragma unroll
        for (int u = 0; u < C::COP; ++u) {
            if (u < ncop && cp[u].on) lds_dma16(cp[u].voff, cp[u].base + (size_t)cp[u].step * (size_t)s, st + cp[u].lds);
        }
    };
    float* terms = reinterpret_cast<float*>(lds + QK_NS * C::STAGE);
    float acc = 0.0f;  // output threadIdx.x: row o / 16, token o % 16
    const int o = (int)threadIdx.x;
    auto fold = [&](int buf) {
        const float* tr = terms + buf * (C::TERMS / 4) + o * QK_SB;
#pragma unroll
        for (int j = 0; j < QK_SLICES; ++j) {
            const float4 v = *reinterpret_cast<const float4*>(tr + 4 * (j ^ (o & 3)));
            acc = (((acc + v.x) + v.y) + v.z) + v.w;
        }
    };
    issue(0);
    const v4i_s z = {0, 0, 0, 0};
    for (int s = 0; s < nst; ++s) {
        wait_vm<0>();    // this wavefront's copies of stage s have landed
        lds_barrier();   // everyone's have; stage s - 1 and the terms of s - 2 are read out
        if (s > 0) fold((s - 1) & 1);
        if (s + 1 < nst) issue(s + 1);
        const uint8_t* st = lds + C::STAGE * (s % QK_NS);
        const uint8_t* wsl = st + C::W_OFF + wave * 16 * C::WL;
        const uint8_t* asl = st + C::A_OFF + wave * 2048;
        // the lane's rows 4 p + i: the slice's four scales each; token c's four scales
        uint2 scw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) scw[i] = *reinterpret_cast<const uint2*>(st + C::SC_OFF + ((4 * p + i) * QK_SB + 4 * wave) * 2);
        const float4 dxv = *reinterpret_cast<const float4*>(st + C::DX_OFF + (c * QK_SB + 4 * wave) * 4);
        const float dx[4] = {dxv.x, dxv.y, dxv.z, dxv.w};
        v4i_s d[QS_S];
#pragma unroll
        for (int j = 0; j < QS_S; ++j) {
            const int ob = qs_slot(c, j, p);
            long a;
            if constexpr (FMT == T_Q8_0) {
                a = *reinterpret_cast<const long*>(wsl + c * C::WL + ob);
            } else {
                const uint2 v = *reinterpret_cast<const uint2*>(wsl + c * C::WL + qs_slot4(c, j, p));
                const int sh = 4 * (p >> 1);
                a = (long)(((uint64_t)q4_signed(v.y, sh) << 32) | (uint64_t)q4_signed(v.x, sh));
            }
            const long b = *reinterpret_cast<const long*>(asl + c * 128 + ob);
            d[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
        }
        float* tw = terms + (s & 1) * (C::TERMS / 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = scw[i].x, hi = scw[i].y;
            float t[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                t[j] = f16_mul_f32(j < 2 ? lo : hi, j & 1, dx[j]) * (float)d[j][i];
            }
            const int oo = (4 * p + i) * 16 + c;  // the output: row 4 p + i, token c
            *reinterpret_cast<float4*>(tw + oo * QK_SB + 4 * (wave ^ (oo & 3))) = make_float4(t[0], t[1], t[2], t[3]);
        }
    }
    lds_barrier();
    fold((nst - 1) & 1);
    const int tk = t0 + (o & 15), r = row0 + (o >> 4);
    if (tk < T && r < n_out) y[(int64_t)tk * n_out + r] = acc;
}

// Whether the K-split GEMM takes the shape: whole 16-block stages, at most 32 tokens (a second
// 16-token tile is a second workgroup on the same rows), 32-bit offsets.
bool gemm_q8_splitk_fits(int ty, int n_out, int k, int T) {
    return T >= 1 && T <= 32 && (k / 32) % QK_SB == 0 && k % 32 == 0 && gemm_q8_staged_fits(ty, n_out, k, T);
}

// Estimated microseconds of the int8 GEMMs, fitted on MI355X timings with the weights read from
// HBM (Q8_0 and Q4_0, 4096 to 14336 rows of 4096 to 14336 values).  K-split: 4.7 + 0.45 (Q4_0)
// or 5.1 + 0.49 (Q8_0) per 16-block stage and workgroup per CU (16 rows x 16 tokens a workgroup,
// 256 CUs).  Staged, up to 32 tokens: a + per 4-block stage 0.49 (Q4_0; a 2.4) or 0.40 (Q8_0;
// a 2.6), 20% more per further workgroup a CU holds (32 rows a workgroup).  Both follow the row
// length, not the token count, while a launch leaves SIMDs idle.
double gemm_splitk_cost_us(int ty, int n_out, int k, int T) {
    const double x = (double)(k / 512) * (double)((n_out + 15) / 16) * (double)((T + 15) / 16) / 256.0;
    return ty == T_Q8_0 ? 5.1 + 0.49 * x : 4.7 + 0.45 * x;
}
double gemm_staged_cost_us(int ty, int n_out, int k) {
    const double wgs_per_cu = (double)(((n_out + 31) / 32 + 255) / 256);
    const bool q8 = ty == T_Q8_0;
    return (q8 ? 2.6 : 2.4) + (q8 ? 0.40 : 0.49) * (double)(k / 128) * (1.0 + 0.2 * (wgs_per_cu - 1.0));
}
// The K-split form where it fits and is estimated faster than the staged one (at 14336 rows of
// 4096 values it is not: 896 workgroups at two per CU run in two rounds).
static bool use_splitk(int ty, int n_out, int k, int T) {
    if (!gemm_q8_splitk_fits(ty, n_out, k, T)) return false;
    return gemm_splitk_cost_us(ty, n_out, k, T) < gemm_staged_cost_us(ty, n_out, k);
}
double gemm_q8_cost_us(int ty, int n_out, int k, int T) {
    if (use_splitk(ty, n_out, k, T)) return gemm_splitk_cost_us(ty, n_out, k, T);
    return gemm_staged_cost_us(ty, n_out, k);
}

template <int FMT>
static void launch_splitk(const uint8_t* W, int n_out, int k, const int8_t* xq, const float* xd, int T, float* y,
                          hipStream_t stream, const uint32_t* active) {
    using C = QkCfg<FMT>;
    // once per process and format, thread-safe (a function-local static); a refusal shows as the
    // launch's error
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemm_q8_splitk<FMT>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
    (void)attr;
    const dim3 grid((unsigned)((n_out + 15) / 16), (unsigned)((T + 15) / 16));
    hipLaunchKernelGGL((k_gemm_q8_splitk<FMT>), grid, dim3(256), (size_t)C::LDS, stream, W, n_out, k, xq, xd, T, y,
                       active);
}

// Whether the staged GEMM takes the shape (Q8_0 or Q4_0 rows): whole stages, 32-bit copy offsets.
bool gemm_q8_staged_fits(int ty, int n_out, int k, int T) {
    const uint64_t nb = (uint64_t)k / 32;
    return (ty == T_Q8_0 || ty == T_Q4_0) && nb % QS_S == 0 && nb > 0 &&
           (uint64_t)n_out * nb * (uint64_t)split_code_bytes(ty) < (1ull << 32) &&
           (uint64_t)T * (uint64_t)k < (1ull << 32);
}

template <int FMT, int TT, int TG>
static void launch_q8_staged(const uint8_t* W, int n_out, int k, const int8_t* xq, const float* xd, int T, float* y,
                             hipStream_t stream, const uint32_t* active) {
    using C = QsCfg<FMT, TT, TG>;
    const dim3 grid((unsigned)((n_out + QS_RW - 1) / QS_RW), (unsigned)((T + C::TW - 1) / C::TW));
    hipLaunchKernelGGL((k_gemm_q8_staged<FMT, TT, TG>), grid, dim3(64 * C::NW), (size_t)(C::STAGE * C::NS), stream,
                       W, n_out, k, xq, xd, T, y, active);
}

// Token tiles: up to 16 tokens one 16-token group; up to 32 two (one wavefront pair of 32 tokens,
// or two pairs of 16); beyond, 64-token workgroups (two pairs of 32 tokens, or four of 16).  A
// wavefront with one 16-token tile does half the work of one with two, so where the launch would
// give a SIMD fewer than QS_TT1_WAVES / 1024 wavefronts of two tiles it takes one-tile wavefronts,
// twice as many.
constexpr uint64_t QS_TT1_WAVES = 2048;

template <int FMT>
static void launch_staged_fmt(const uint8_t* W, int n_out, int k, const int8_t* xq, const float* xd, int T, float* y,
                              hipStream_t stream, const uint32_t* active) {
    const uint64_t row_wgs = (uint64_t)(n_out + QS_RW - 1) / QS_RW;
    if (T <= 16) {
        launch_q8_staged<FMT, 1, 1>(W, n_out, k, xq, xd, T, y, stream, active);
    } else if (T <= 32) {
        if (row_wgs * 2 < QS_TT1_WAVES)
            launch_q8_staged<FMT, 1, 2>(W, n_out, k, xq, xd, T, y, stream, active);
        else
            launch_q8_staged<FMT, 2, 1>(W, n_out, k, xq, xd, T, y, stream, active);
    } else {
        if (row_wgs * (uint64_t)((T + 63) / 64) * 4 < QS_TT1_WAVES)
            launch_q8_staged<FMT, 1, 4>(W, n_out, k, xq, xd, T, y, stream, active);
        else
            launch_q8_staged<FMT, 2, 2>(W, n_out, k, xq, xd, T, y, stream, active);
    }
}

// Q8_0 rows of any shape (the staged GEMM where it fits, else the register-staged one); Q4_0 rows
// where the staged GEMM fits (gemm_q8_staged_fits).
void launch_gemm_q8_split(int ty, const uint8_t* W, int n_out, int k, const uint8_t* ws, int T, float* y,
                          hipStream_t stream, const uint32_t* active) {
    const ActLayout L = act_layout(ACT_Q8_0, (uint64_t)T, (uint64_t)k);
    const int8_t* xq = reinterpret_cast<const int8_t*>(ws + L.codes);
    const float* xd = reinterpret_cast<const float*>(ws + L.d);
    if (use_splitk(ty, n_out, k, T)) {  // rows of whole 16-block stages, up to 32 tokens
        if (ty == T_Q4_0)
            launch_splitk<T_Q4_0>(W, n_out, k, xq, xd, T, y, stream, active);
        else
            launch_splitk<T_Q8_0>(W, n_out, k, xq, xd, T, y, stream, active);
        return;
    }
    if (ty == T_Q4_0) {
        launch_staged_fmt<T_Q4_0>(W, n_out, k, xq, xd, T, y, stream, active);
        return;
    }
    if (gemm_q8_staged_fits(T_Q8_0, n_out, k, T)) {
        launch_staged_fmt<T_Q8_0>(W, n_out, k, xq, xd, T, y, stream, active);
        return;
    }
    // other shapes: the register-staged kernel; up to 64 tokens: 16-token tiles; beyond, 32-token tiles (a token tile per wavefront, up to
    // four wavefronts on the same 16 rows)
    const int TT = T <= 64 ? 1 : 2;
    const int tiles = (T + 16 * TT - 1) / (16 * TT);
    const int wpw = tiles < 4 ? tiles : 4;
    const dim3 grid((unsigned)((n_out + 15) / 16), (unsigned)((tiles + wpw - 1) / wpw));
    const bool vec = (k / 32) % (2 * GQ_G) == 0;
    const dim3 block(64 * wpw);
    if (TT == 1 && vec)
        hipLaunchKernelGGL((k_gemm_q8_split<1, true>), grid, block, 0, stream, W, n_out, k, xq, xd, T, y, active);
    else if (TT == 1)
        hipLaunchKernelGGL((k_gemm_q8_split<1, false>), grid, block, 0, stream, W, n_out, k, xq, xd, T, y, active);
    else if (vec)
        hipLaunchKernelGGL((k_gemm_q8_split<2, true>), grid, block, 0, stream, W, n_out, k, xq, xd, T, y, active);
    else
        hipLaunchKernelGGL((k_gemm_q8_split<2, false>), grid, block, 0, stream, W, n_out, k, xq, xd, T, y, active);
}

}  // namespace syn
