// MoeGrouped over Q8_0 experts on gfx950 (crates/kernels-cpu/src/moe.rs:470-551 with
// WeightType::Q8_0, crates/kernels-cpu/src/moe/entry.rs:50-55): every entry (a packed slot) of
// expert e takes its row of x, quantized to Q8_0 (act.rs:323-342); gate and up are two Gemv
// values over the expert's matrices, h = silu(g) * u rounded once; h is quantized to Q8_0 and the
// down Gemv's row goes to the entry's slot.  Each Gemv value is the reference's: per 32-value
// block the exact I32 sum s and the term (dw * dx) * s, the terms added in ascending block order
// from +0.0 (gemv.rs:539-547, portable.rs:114-190).
//
// Mapping.  A workgroup takes one expert and 64 output rows (four wavefronts of 16 rows; four
// lanes per row take the row's blocks in turn, block b to lane b mod 4, and hand the running
// sum on with a DPP rotation, so the fold stays in block order).  It walks the expert's entries
// eight at a time; each pass streams the rows' weights once, 16 blocks per stage through a
// per-wavefront LDS stage read with 16-byte loads.  Gate and up are staged side by side, so one
// pass forms both dots of every entry and h directly.  Empty experts (and experts a site mask
// leaves out, which the packing leaves empty) exit at once.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

constexpr int MQ_P = 4;                 // lanes per output row
constexpr int MQ_G = 64 / MQ_P;         // rows per wavefront
constexpr int MQ_C = 16;                // blocks per row per stage
constexpr int MQ_BB = 34;               // bytes per Q8_0 block
constexpr int MQ_SEG = MQ_C * MQ_BB;    // bytes per row per stage
constexpr int MQ_STAGE = MQ_G * MQ_SEG + 64;
constexpr int MQ_R = 8;                 // entries per pass

// Gather + Q8_0: entry i (packed order, i < *total) takes row slots[i] / top_k of x (gather) or
// row i of x.  Eight lanes per 32-value block; codes [entries][k], scales [entries][k / 32].
__global__ __launch_bounds__(256) void k_moe_gather_q8_0(const float* __restrict__ x,
                                                         const uint32_t* __restrict__ slots, int nentries,
                                                         int top_k, int k, const uint32_t* __restrict__ err,
                                                         int8_t* __restrict__ codes, float* __restrict__ dout,
                                                         int gather, const uint32_t* __restrict__ total) {
    if (err[0]) return;
    const int nb = k / 32;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t blk = t >> 3;
    const int sub = threadIdx.x & 7;
    const uint64_t entry = blk / (uint64_t)nb;
    const int b = (int)(blk - entry * (uint64_t)nb);
    const bool live = entry < (uint64_t)nentries && entry < (uint64_t)*total;  // uniform per block
    float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        const uint64_t row = gather ? slots[entry] / (uint32_t)top_k : entry;
        v4 = reinterpret_cast<const float4*>(x + row * (uint64_t)k + (uint64_t)b * 32)[sub];
    }
    const Q8_0Lane r = q8_0_block_lane(v4);
    if (!live) return;
    reinterpret_cast<uint32_t*>(codes + entry * (uint64_t)k + (uint64_t)b * 32)[sub] = r.packed;
    if (sub == 0) dout[entry * (uint64_t)nb + b] = r.d;
}

void launch_moe_gather_q8_0(const float* x, const uint32_t* slots, int nentries, int top_k, int k,
                            const uint32_t* err, int8_t* codes, float* d, int gather, const uint32_t* total,
                            hipStream_t stream) {
    const uint64_t threads = (uint64_t)nentries * (k / 32) * 8;
    if (threads == 0) return;
    hipLaunchKernelGGL(k_moe_gather_q8_0, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, x, slots,
                       nentries, top_k, k, err, codes, d, gather, total);
}

// The code dwords and the F16 scale of the Q8_0 block at `blk` (2-byte aligned) in LDS.
SYN_DEV void q8_0_block_at(const uint8_t* blk, uint32_t& dw16, uint32_t qs[8]) {
    const int odd = ((uintptr_t)blk & 2) != 0;
    const uint32_t* base = reinterpret_cast<const uint32_t*>(blk - (odd ? 2 : 0));
    uint32_t w[10];
#pragma unroll
    for (int i = 0; i < 10; ++i) w[i] = base[i];
    dw16 = odd ? (w[0] >> 16) : (w[0] & 0xFFFFu);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = odd ? w[i + 1] : w[i];
        const uint32_t hi = odd ? w[i + 2] : w[i + 1];
        qs[i] = __builtin_amdgcn_alignbyte(hi, lo, odd ? 0u : 2u);
    }
}

// (dw * dx) * s of one block against one entry's Q8_0 codes (16-byte aligned) and scale.
SYN_DEV float q8_0_term(uint32_t dw16, const uint32_t qs[8], const int8_t* __restrict__ xq, float dx) {
    const uint4 x0 = reinterpret_cast<const uint4*>(xq)[0], x1 = reinterpret_cast<const uint4*>(xq)[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    int s = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) s = sdot4(qs[t], xw[t], s);
    return (f16_to_f32(dw16) * dx) * (float)s;
}

// MODE 0: gate (w0) and up (w1), n_out = inter rows of k = hidden, h[entry][inter] = silu(g) u.
// MODE 1: down (w0), n_out = hidden rows of k = inter, out[slot][hidden].
template <int MODE, int VEC>
__global__ __launch_bounds__(256) void k_moe_q8(const uint8_t* __restrict__ w0all, const uint8_t* __restrict__ w1all,
                                                uint64_t mat_bytes, int n_out, int k,
                                                const uint32_t* __restrict__ offsets,
                                                const uint32_t* __restrict__ slots,
                                                const uint32_t* __restrict__ err,
                                                const int8_t* __restrict__ aq, const float* __restrict__ ad,
                                                float* __restrict__ y) {
    constexpr int NM = MODE == 0 ? 2 : 1;
    if (err[0]) return;
    const int e = blockIdx.y;
    const uint32_t e0 = offsets[e], ne = offsets[e + 1] - e0;
    if (ne == 0) return;  // uniform
    __shared__ __attribute__((aligned(16))) uint8_t stage_all[4][NM][MQ_STAGE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane / MQ_P, j = lane % MQ_P;
    const int row0 = (blockIdx.x * 4 + wave) * MQ_G;
    const int row = row0 + g;
    const int nb = k / 32;
    const int64_t row_bytes = (int64_t)nb * MQ_BB;
    const uint8_t* wm[2] = {w0all + (uint64_t)e * mat_bytes, MODE == 0 ? w1all + (uint64_t)e * mat_bytes : nullptr};
    for (uint32_t c0 = 0; c0 < ne; c0 += MQ_R) {  // uniform
        const int rows = ne - c0 < (uint32_t)MQ_R ? (int)(ne - c0) : MQ_R;
        const int8_t* xq = aq + (uint64_t)(e0 + c0) * k;
        const float* xd = ad + (uint64_t)(e0 + c0) * nb;
        float acc[NM][MQ_R];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < MQ_R; ++r) acc[m][r] = 0.0f;
        for (int cb = 0; cb < nb; cb += MQ_C) {
            const int nblk = nb - cb < MQ_C ? nb - cb : MQ_C;
            const int seg = nblk * MQ_BB;
#pragma unroll
            for (int m = 0; m < NM; ++m)
                for (int gg = 0; gg < MQ_G; ++gg) {
                    if (row0 + gg >= n_out) break;
                    const uint8_t* src = wm[m] + (int64_t)(row0 + gg) * row_bytes + (int64_t)cb * MQ_BB;
                    uint8_t* dst = stage_all[wave][m] + gg * MQ_SEG;
                    if constexpr (VEC == 16) {
                        typedef unsigned int v4u __attribute__((ext_vector_type(4)));
                        for (int p = lane; p < seg / 16; p += 64)
                            *reinterpret_cast<v4u*>(dst + 16 * p) =
                                __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + 16 * p));
                        // the segment's tail when seg is not a multiple of 16 (a partial stage)
                        for (int p = (seg / 16) * 16 + lane; p < seg; p += 64) dst[p] = src[p];
                    } else {
                        for (int p = lane; p < seg; p += 64) dst[p] = src[p];
                    }
                }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < MQ_C / MQ_P; ++u) {
                const int bi = u * MQ_P + j;
                const bool valid = bi < nblk && row < n_out;
                float t[NM][MQ_R];
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < MQ_R; ++r) t[m][r] = 0.0f;
                if (valid) {
                    const int b = cb + bi;
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        uint32_t dw16, qs[8];
                        q8_0_block_at(stage_all[wave][m] + g * MQ_SEG + bi * MQ_BB, dw16, qs);
#pragma unroll
                        for (int r = 0; r < MQ_R; ++r)
                            if (r < rows) t[m][r] = q8_0_term(dw16, qs, xq + (int64_t)r * k + b * 32, xd[r * nb + b]);
                    }
                }
                // in-order fold: the running sum visits the row's four lanes in turn
#pragma unroll
                for (int s = 0; s < MQ_P; ++s)
#pragma unroll
                    for (int m = 0; m < NM; ++m)
#pragma unroll
                        for (int r = 0; r < MQ_R; ++r) {
                            acc[m][r] = rot1<MQ_P>(acc[m][r]);
                            acc[m][r] = acc[m][r] + ((j == s) ? t[m][r] : 0.0f);
                        }
            }
            __syncthreads();
        }
        if (j == MQ_P - 1 && row < n_out) {
#pragma unroll
            for (int r = 0; r < MQ_R; ++r) {
                if (r >= rows) break;
                const uint32_t entry = e0 + c0 + r;
                if constexpr (MODE == 0)
                    y[(uint64_t)entry * n_out + row] = ref_silu(acc[0][r]) * acc[1][r];
                else
                    y[(uint64_t)slots[entry] * n_out + row] = acc[0][r];
            }
        }
    }
}

void launch_moe_q8(int mode, const uint8_t* w0, const uint8_t* w1, uint64_t mat_bytes, int n_experts, int n_out,
                   int k, const uint32_t* offsets, const uint32_t* slots, const uint32_t* err, const int8_t* aq,
                   const float* ad, float* y, hipStream_t stream) {
    const dim3 grid((unsigned)((n_out + 4 * MQ_G - 1) / (4 * MQ_G)), (unsigned)n_experts);
    const bool vec = ((uintptr_t)w0 % 16 == 0) && (!w1 || (uintptr_t)w1 % 16 == 0) &&
                     ((int64_t)(k / 32) * MQ_BB) % 16 == 0 && mat_bytes % 16 == 0;
    if (mode == 0) {
        if (vec)
            hipLaunchKernelGGL((k_moe_q8<0, 16>), grid, dim3(256), 0, stream, w0, w1, mat_bytes, n_out, k, offsets,
                               slots, err, aq, ad, y);
        else
            hipLaunchKernelGGL((k_moe_q8<0, 1>), grid, dim3(256), 0, stream, w0, w1, mat_bytes, n_out, k, offsets,
                               slots, err, aq, ad, y);
    } else {
        if (vec)
            hipLaunchKernelGGL((k_moe_q8<1, 16>), grid, dim3(256), 0, stream, w0, w1, mat_bytes, n_out, k, offsets,
                               slots, err, aq, ad, y);
        else
            hipLaunchKernelGGL((k_moe_q8<1, 1>), grid, dim3(256), 0, stream, w0, w1, mat_bytes, n_out, k, offsets,
                               slots, err, aq, ad, y);
    }
}

}  // namespace syn
