// Doorbells on gfx950: the device's halves of the host <-> device flags of one step
// (plan/rfcs/RFC-0040-kernel-providers-and-backends.md:545-590; crates/kernels/src/provider.rs:346-377).
//
// A flag is a 4-byte word on a 64-byte line of its own in pinned, fine-grained host pages.
//  * signal: one lane stores the value at system scope, with release order, after the work the
//    stream ran before it: the payload is visible before the flag.
//  * wait: one lane polls the flag at system scope with acquire order and a sleep between polls
//    until it compares equal (or greater or equal) to the value, then stores the reset value
//    when asked (the consumer reset of the constant-valued handshake).  The wait is bounded: past
//    `max_ticks` of the device's constant-rate wall clock it stops without the reset and records
//    `tag` in the status word (the first timeout wins), so the stream always drains and the host
//    reports the stall.  These are the RFC's store and spin kernels; they capture into a graph as
//    plain kernel nodes with their values fixed, as the handshake requires.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

__global__ __launch_bounds__(64) void k_bell_signal(uint32_t* flag, uint32_t value) {
    if (threadIdx.x == 0) __hip_atomic_store(flag, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(64) void k_bell_wait(uint32_t* flag, uint32_t value, int geq, int has_reset,
                                                  uint32_t reset, uint64_t max_ticks, uint32_t* status,
                                                  uint32_t tag) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = wall_clock64();
    for (;;) {
        const uint32_t v = __hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
        if (geq ? v >= value : v == value) {
            if (has_reset) __hip_atomic_store(flag, reset, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        if (wall_clock64() - t0 > max_ticks) {
            uint32_t none = 0;
            __hip_atomic_compare_exchange_strong(status, &none, tag, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        __builtin_amdgcn_s_sleep(16);
    }
}

void launch_bell_signal(uint32_t* flag, uint32_t value, hipStream_t stream) {
    hipLaunchKernelGGL(k_bell_signal, dim3(1), dim3(64), 0, stream, flag, value);
}

void launch_bell_wait(uint32_t* flag, uint32_t value, int geq, int has_reset, uint32_t reset, uint64_t max_ticks,
                      uint32_t* status, uint32_t tag, hipStream_t stream) {
    hipLaunchKernelGGL(k_bell_wait, dim3(1), dim3(64), 0, stream, flag, value, geq, has_reset, reset, max_ticks,
                       status, tag);
}

}  // namespace syn
