// RmsNorm on gfx950 (crates/kernels/src/reference/norm.rs:39-47), the first half of Logits
// (crates/kernels/src/reference/linear.rs:118-161):
//   ss = sum of x[i] x[i] in the F32Fixed order; mean = ss / n; scale = 1 / sqrt(mean + eps);
//   y[i] = (x[i] scale) g[i]
// each step one IEEE F32 operation (the library compiles without contraction, with correctly
// rounded division and square root).
//
// One workgroup per row.  The F32Fixed order (crates/kernels/src/reference/reduce.rs:7-20) is
// blocks of 32 terms summed sequentially from +0.0, then the block sums added pairwise, level by
// level, an odd last sum carried up unchanged: each lane sums whole blocks, and the levels run
// through LDS.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAX_BLOCKS = NORM_MAX_COLS / 32;
static_assert(NORM_MAX_BLOCKS / 2 <= NORM_THREADS, "one pair per thread per level");

__global__ __launch_bounds__(NORM_THREADS) void k_rms_norm(const float* __restrict__ x, const float* __restrict__ g,
                                                          int n, float eps, float* __restrict__ y,
                                                          const uint32_t* __restrict__ active) {
    const int row = blockIdx.x;
    if (active && row >= active_rows(active, 0, (int)gridDim.x)) return;
    __shared__ float sums[NORM_MAX_BLOCKS];
    const float* xr = x + (int64_t)row * n;
    const int nblocks = (n + 31) / 32;
    for (int b = threadIdx.x; b < nblocks; b += NORM_THREADS) {
        const int end = (b + 1) * 32 < n ? (b + 1) * 32 : n;
        float acc = 0.0f;
        for (int i = b * 32; i < end; ++i) acc = acc + xr[i] * xr[i];
        sums[b] = acc;
    }
    __syncthreads();
    // NORM_MAX_BLOCKS / 2 <= NORM_THREADS: one pair per thread at every level
    for (int m = nblocks; m > 1; m = (m + 1) / 2) {
        const int half = m / 2, i = threadIdx.x;
        const bool odd = (m & 1) && i == 0;
        float v = 0.0f, carry = 0.0f;
        if (i < half) v = sums[2 * i] + sums[2 * i + 1];
        if (odd) carry = sums[m - 1];  // the odd last sum moves to index `half` unchanged
        __syncthreads();
        if (i < half) sums[i] = v;
        if (odd) sums[half] = carry;
        __syncthreads();
    }
    const float ss = nblocks ? sums[0] : 0.0f;
    const float mean = ss / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    float* yr = y + (int64_t)row * n;
    for (int i = threadIdx.x; i < n; i += NORM_THREADS) yr[i] = (xr[i] * scale) * g[i];
}

void launch_rms_norm(const float* x, const float* g, int rows, int n, float eps, float* y, hipStream_t stream,
                     const uint32_t* active) {
    if (rows == 0 || n == 0) return;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(NORM_THREADS), 0, stream, x, g, n, eps, y, active);
}

}  // namespace syn
