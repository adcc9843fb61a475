// Measurement helper: a read-only HBM stream with the decode GEMV's load pattern (16-byte
// non-temporal loads, nine per lane, each wavefront instruction covering whole 128-byte lines),
// so the HBM byte counters can be calibrated on a kernel of known traffic.  Not on the op path.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef unsigned int v4u_p __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_hbm_read_probe(const uint8_t* __restrict__ src, uint64_t nchunks,
                                                        uint32_t* __restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * 256 * 9;
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 9; ++i) {
        const uint64_t c = base + (uint64_t)i * 256 + threadIdx.x;
        if (c < nchunks) {
            const v4u_p v = __builtin_nontemporal_load(reinterpret_cast<const v4u_p*>(src + 16 * c));
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    // one word per workgroup (the reads cannot be dropped; the write is 4 bytes per 36 KiB read)
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int i = 0; i < 256; ++i) r ^= red[i];
        sink[blockIdx.x] = r;
    }
}

void launch_hbm_read_probe(const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream) {
    const uint64_t nchunks = bytes / 16;
    const uint64_t wg = (nchunks + 256 * 9 - 1) / (256 * 9);
    if (wg == 0) return;
    hipLaunchKernelGGL(k_hbm_read_probe, dim3((unsigned)wg), dim3(256), 0, stream, src, nchunks, sink);
}

}  // namespace syn
