// Self-check of the quantizers' short forms (common.hpp: div127, recip_rn, neg127_div, f16_round,
// nearest_int_small) against the correctly rounded F32 division, the integer F16 conversion and
// the reference's nearest_int, over every F32 bit pattern.  Not on the op path; a GPU test runs it.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

constexpr int DIVCHK_PER = 256;  // patterns a thread
constexpr int DIVCHK_TPB = 256;

__global__ __launch_bounds__(DIVCHK_TPB) void k_div_forms_check(unsigned long long* __restrict__ counts) {
    __shared__ uint32_t c[5];
    if (threadIdx.x < 5) c[threadIdx.x] = 0;
    __syncthreads();
    uint32_t n[5] = {0, 0, 0, 0, 0};
    const uint32_t base = ((uint32_t)blockIdx.x * DIVCHK_TPB + threadIdx.x) * DIVCHK_PER;
    for (int i = 0; i < DIVCHK_PER; ++i) {
        const uint32_t bits = base + (uint32_t)i;
        const uint32_t mag = bits & 0x7FFFFFFFu;
        if (mag > 0x7F800000u) continue;  // NaN
        const float x = u2f(bits);
        if (bits < 0x7F800000u) n[0] += f2u(div127(x)) != f2u(x / 127.0f);  // finite, >= 0
        n[1] += f2u(recip_rn(x)) != f2u(1.0f / x);
        n[2] += f2u(neg127_div(x)) != f2u(-127.0f / x);
        n[3] += f2u(f16_round(x)) != f2u(f16_to_f32(f16_bits(x)));
        if (mag < 0x4A000000u) n[4] += nearest_int_small(x) != nearest_int(x);  // |x| < 2^21
    }
#pragma unroll
    for (int k = 0; k < 5; ++k)
        if (n[k]) atomicAdd(&c[k], n[k]);
    __syncthreads();
    if (threadIdx.x < 5 && c[threadIdx.x]) atomicAdd(&counts[threadIdx.x], (unsigned long long)c[threadIdx.x]);
}

void launch_div_forms_check(unsigned long long* counts, hipStream_t stream) {
    const unsigned grid = (unsigned)((1ull << 32) / ((uint64_t)DIVCHK_TPB * DIVCHK_PER));
    hipLaunchKernelGGL(k_div_forms_check, dim3(grid), dim3(DIVCHK_TPB), 0, stream, counts);
}

}  // namespace syn
