// Measurement helper: a read-only HBM stream with the decode GEMV's load pattern (16-byte
// non-temporal loads, each wavefront instruction covering whole 128-byte lines), so the HBM byte
// counters can be calibrated on a kernel of known traffic, and so a lone op can be set against a
// bare read of its bytes.  Nine loads per lane from 256 MiB (the calibration read); one below,
// the fastest shape at decode sizes (9.4 MB in 2.8 us against 5.8 us at nine per lane).  Not on
// the op path.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

typedef unsigned int v4u_p __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void k_hbm_read_probe(const uint8_t* __restrict__ src, uint64_t nchunks,
                                                        uint32_t* __restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * 256 * U;
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const uint64_t c = base + (uint64_t)i * 256 + threadIdx.x;
        if (c < nchunks) {
            const v4u_p v = __builtin_nontemporal_load(reinterpret_cast<const v4u_p*>(src + 16 * c));
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    // one word per workgroup (the reads cannot be dropped; the write is 4 bytes per 256 U chunks):
    // each wavefront's xor by lane swaps, then the four wavefronts' words
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// The decode GEMV's wavefront pattern over X8 weights: a wavefront reads 9,216 bytes (eight
// 1,152-byte runs) with nine loads a lane, instruction i reading line i of every run; WAVES
// wavefronts a workgroup.  Each wavefront writes one word (its unit's) to sink.
template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_hbm_read_runs(const uint8_t* __restrict__ src, uint64_t bytes,
                                                              uint32_t* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    const uint64_t unit = (uint64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
    const uint64_t base = unit * 9216 + (uint64_t)(lane >> 3) * 1152 + 16 * (uint64_t)(lane & 7);
    uint32_t acc = 0;
    v4u_p v[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) {
        const uint64_t off = base + 128 * (uint64_t)i;
        v[i] = off < bytes ? __builtin_nontemporal_load(reinterpret_cast<const v4u_p*>(src + off)) : v4u_p{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 9; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m);
    if (lane == 0 && unit * 9216 < bytes) sink[unit] = acc;
}

uint64_t hbm_read_runs_units(uint64_t bytes) { return (bytes + 9215) / 9216; }

void launch_hbm_read_runs(int waves, const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream) {
    const uint64_t units = hbm_read_runs_units(bytes);
    if (units == 0) return;
    if (waves == 1)
        hipLaunchKernelGGL(k_hbm_read_runs<1>, dim3((unsigned)units), dim3(64), 0, stream, src, bytes, sink);
    else
        hipLaunchKernelGGL(k_hbm_read_runs<8>, dim3((unsigned)((units + 7) / 8)), dim3(512), 0, stream, src, bytes,
                           sink);
}

int hbm_read_probe_loads(uint64_t bytes) { return bytes >= (256ull << 20) ? 9 : 1; }

uint64_t hbm_read_probe_workgroups(uint64_t bytes) {
    const uint64_t per = 256ull * (uint64_t)hbm_read_probe_loads(bytes);
    return (bytes / 16 + per - 1) / per;
}

void launch_hbm_read_probe(const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream) {
    const uint64_t nchunks = bytes / 16;
    const uint64_t wg = hbm_read_probe_workgroups(bytes);
    if (wg == 0) return;
    if (hbm_read_probe_loads(bytes) == 9)
        hipLaunchKernelGGL(k_hbm_read_probe<9>, dim3((unsigned)wg), dim3(256), 0, stream, src, nchunks, sink);
    else
        hipLaunchKernelGGL(k_hbm_read_probe<1>, dim3((unsigned)wg), dim3(256), 0, stream, src, nchunks, sink);
}

}  // namespace syn
