// Activation quantization on gfx950: F32 rows -> the 8-bit blocks the GEMV kernels read.
//
// Q8_0 follows crates/kernels-cpu/src/gemv/act.rs:323-342 (ggml's arm64 quantizer, ties to
// even, F16-rounded scale); Q8_K follows act.rs:351-373 (signed maximum, first on ties,
// ggml's nearest_int).  A block holding a NaN or an infinity gets scale NaN and zero codes.
// Both kernels also write the exact I32 sum of every 32 codes.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

__global__ __launch_bounds__(256) void k_quant_q8k(const float* __restrict__ x, uint64_t nblk,
                                                   int8_t* __restrict__ codes,
                                                   float* __restrict__ dout,
                                                   int32_t* __restrict__ sums) {
    const uint64_t blk = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;
    q8k_block_wave(x + blk * 256, codes + blk * 256, dout + blk, sums + blk * 8, threadIdx.x & 63);
}

// Eight lanes per 32-value block, eight blocks per wavefront.
__global__ __launch_bounds__(256) void k_quant_q8_0(const float* __restrict__ x, uint64_t nblk,
                                                    int8_t* __restrict__ codes,
                                                    float* __restrict__ dout,
                                                    int32_t* __restrict__ sums) {
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t blk = t >> 3;
    const int sub = threadIdx.x & 7;
    const bool live = blk < nblk;
    float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v4 = reinterpret_cast<const float4*>(x + blk * 32)[sub];
    const Q8_0Lane r = q8_0_block_lane(v4);
    if (!live) return;
    reinterpret_cast<uint32_t*>(codes + blk * 32)[sub] = r.packed;
    if (sub == 0) {
        sums[blk] = r.sum;
        dout[blk] = r.d;
    }
}

// Several single rows at once: problem p takes workgroups [wg_begin[p], wg_begin[p+1]), one
// wavefront per 256-value block, each into its own workspace.
struct QuantBatch {
    const float* x[SYN_BATCH];
    uint8_t* ws[SYN_BATCH];
    int nblk[SYN_BATCH];
    int wg_begin[SYN_BATCH + 1];
    int np;
};

__global__ __launch_bounds__(256) void k_quant_q8k_batch(QuantBatch qb) {
    int p = 0;
    while (p + 1 < qb.np && (int)blockIdx.x >= qb.wg_begin[p + 1]) ++p;
    const int blk = ((int)blockIdx.x - qb.wg_begin[p]) * 4 + (threadIdx.x >> 6);
    const int nblk = qb.nblk[p];
    if (blk >= nblk) return;
    const ActLayout L = act_layout(ACT_Q8K, 1, (uint64_t)nblk * 256);
    uint8_t* ws = qb.ws[p];
    q8k_block_wave(qb.x[p] + (int64_t)blk * 256, reinterpret_cast<int8_t*>(ws + L.codes) + (int64_t)blk * 256,
                   reinterpret_cast<float*>(ws + L.d) + blk,
                   reinterpret_cast<int32_t*>(ws + L.sums) + (int64_t)blk * 8, threadIdx.x & 63);
}

void launch_act_quant_batch(int np, const float* const* x, const int* k, uint8_t* const* ws,
                            hipStream_t stream) {
    QuantBatch qb{};
    qb.np = np;
    int wg = 0;
    for (int p = 0; p < np; ++p) {
        qb.x[p] = x[p];
        qb.ws[p] = ws[p];
        qb.nblk[p] = k[p] / 256;
        qb.wg_begin[p] = wg;
        wg += (qb.nblk[p] + 3) / 4;
    }
    qb.wg_begin[np] = wg;
    if (wg == 0) return;
    hipLaunchKernelGGL(k_quant_q8k_batch, dim3(wg), dim3(256), 0, stream, qb);
}

// The Q8_0 kernel leaves no per-32 sums for Q8_K; Q8_K's sums come from its own kernel.
void launch_act_quant(int kind, const float* x, uint64_t rows, uint64_t k, uint8_t* ws,
                      hipStream_t stream) {
    const ActLayout L = act_layout(kind, rows, k);
    int8_t* codes = reinterpret_cast<int8_t*>(ws + L.codes);
    float* d = reinterpret_cast<float*>(ws + L.d);
    int32_t* sums = reinterpret_cast<int32_t*>(ws + L.sums);
    const uint64_t n = rows * k;
    if (kind == ACT_Q8K) {
        const uint64_t nblk = n / 256;
        if (nblk == 0) return;
        hipLaunchKernelGGL(k_quant_q8k, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, stream, x,
                           nblk, codes, d, sums);
    } else if (kind == ACT_Q8_0) {
        const uint64_t nblk = n / 32;
        if (nblk == 0) return;
        hipLaunchKernelGGL(k_quant_q8_0, dim3((unsigned)((nblk + 31) / 32)), dim3(256), 0, stream,
                           x, nblk, codes, d, sums);
    }
}

}  // namespace syn
