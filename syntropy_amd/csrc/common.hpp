// Device helpers shared by the gfx950 kernels of the quantized-matmul path.
//
// Every float operation here is one IEEE F32 operation: the library is compiled with
// -ffp-contract=off, correctly rounded division and square root, and F32/F16 denormals kept,
// so each helper gives the same bits as the reference function it cites.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "layout.hpp"

#define SYN_DEV __device__ __forceinline__

namespace syn {

constexpr int WAVE = 64;

SYN_DEV uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
SYN_DEV float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
SYN_DEV bool finite_f(float v) { return (f2u(v) & 0x7F800000u) != 0x7F800000u; }

// Exact F16 -> F32 (v_cvt_f32_f16 with F16 denormals kept): the value of
// crates/kernels/src/reference/act_quant.rs:448-467 for every non-NaN pattern.
SYN_DEV float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// F32 -> F16 bits, round to nearest even with subnormals, NaN -> sign|0x7E00
// (crates/kernels/src/reference/act_quant.rs:400-446), in integer arithmetic.
SYN_DEV uint32_t f16_bits(float x) {
    uint32_t b = f2u(x);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t a = b & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    int e = (int)(a >> 23) - 127;
    uint32_t mant = a & 0x007FFFFFu;
    if (e >= -14) {
        uint32_t base = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (base & 1u))) base += 1;
        return sign | base;
    }
    if (a < 0x00800000u) return sign;
    uint32_t shift = (uint32_t)(-e - 1);
    if (shift >= 40) return sign;
    uint64_t sig = (uint64_t)(mant | 0x00800000u);
    uint64_t base = sig >> shift;
    uint64_t r = sig & ((1ull << shift) - 1);
    uint64_t h = 1ull << (shift - 1);
    if (r > h || (r == h && (base & 1))) base += 1;
    return sign | (uint32_t)base;
}

// ggml's nearest_int (ggml-quants.c:621-626; kernels-cpu/src/gemv/act.rs:345-348).
// The quantizers' correctly rounded F32 divisions in fewer instructions than the compiler's
// general sequence (about ten each).  Each form equals the division bit for bit over its whole
// domain on gfx950; syn_div_forms_check compares them over every F32 pattern.
//  div127(a), a finite and >= 0: RN(a * RN(1/127)) and one fma residual step (Markstein).
SYN_DEV float div127(float a) {
    const float y = 1.0f / 127.0f;
    const float q = a * y;
    return __builtin_fmaf(__builtin_fmaf(-q, 127.0f, a), y, q);
}
//  recip_rn(b): v_rcp_f32 and one fma Newton step where 2^-126 <= |b| < 2^126, else the division.
SYN_DEV float recip_rn(float b) {
    const uint32_t m = f2u(b) & 0x7FFFFFFFu;
    if (m >= 0x00800000u && m < 0x7E800000u) {
        const float y = __builtin_amdgcn_rcpf(b);
        return __builtin_fmaf(__builtin_fmaf(-b, y, 1.0f), y, y);
    }
    return 1.0f / b;
}
//  neg127_div(b) = -127 / b: RN(-127 * recip) and one fma residual step where 2^-120 <= |b| <
//  2^126, else the division.
SYN_DEV float neg127_div(float b) {
    const uint32_t m = f2u(b) & 0x7FFFFFFFu;
    if (m >= 0x03800000u && m < 0x7E800000u) {
        const float y = __builtin_amdgcn_rcpf(b);
        const float r = __builtin_fmaf(__builtin_fmaf(-b, y, 1.0f), y, y);
        const float q = -127.0f * r;
        return __builtin_fmaf(__builtin_fmaf(-q, b, -127.0f), r, q);
    }
    return -127.0f / b;
}
// F32 -> F16 -> F32 by the hardware conversions (round to nearest even, F16 subnormals kept):
// f16_to_f32(f16_bits(x)) for every non-NaN x (also checked by syn_div_forms_check).
SYN_DEV float f16_round(float x) { return (float)(_Float16)x; }

SYN_DEV int nearest_int(float f) {
    float v = f + 12582912.f;
    return (int)(f2u(v) & 0x007FFFFFu) - 0x00400000;
}
// nearest_int(f) for |f| < 2^21 (where f + 1.5 * 2^23 rounds f to the nearest even integer, in
// its low bits; just below 2^22 the sum rounds up to 2^24 and the two part): v_rndne_f32 and a
// conversion (syn_div_forms_check compares the two over every such f).
SYN_DEV int nearest_int_small(float f) { return (int)__builtin_rintf(f); }

// get_scale_min_k4 (crates/kernels-cpu/src/gemv.rs:528-537) from the 12 packed bytes held in
// three little-endian words.
SYN_DEV void scales_k4(uint32_t w0, uint32_t w1, uint32_t w2, int* sc, int* mn) {
    // bytes q[0..3] = w0, q[4..7] = w1, q[8..11] = w2
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t qj = (w0 >> (8 * j)) & 0xFFu;
        uint32_t qj4 = (w1 >> (8 * j)) & 0xFFu;
        uint32_t qj8 = (w2 >> (8 * j)) & 0xFFu;
        sc[j] = (int)(qj & 63u);
        mn[j] = (int)(qj4 & 63u);
        sc[j + 4] = (int)((qj8 & 0xFu) | ((qj >> 6) << 4));
        mn[j + 4] = (int)((qj8 >> 4) | ((qj4 >> 6) << 4));
    }
}

// The reference's software exp (crates/kernels/src/reference/math.rs:45-75).
SYN_DEV float pow2i(int k) { return u2f((uint32_t)(k + 127) << 23); }
SYN_DEV float ref_exp(float x) {
    const float LOG2_E = 1.44269504088896340736f;
    const float LN2_HI = __builtin_bit_cast(float, 0x3F317200u);
    const float LN2_LO = 1.4286068e-6f;
    if (x != x) return x + x;
    if (x > 88.72284f) return __builtin_inff();
    if (x < -103.97208f) return 0.0f;
    float kf = __builtin_rintf(x * LOG2_E);
    float r = (x - kf * LN2_HI) - kf * LN2_LO;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    int k = (int)kf;
    int k1 = k >> 1;  // floor division by 2 (Rust div_euclid(2)): arithmetic shift
    return (p * pow2i(k1)) * pow2i(k - k1);
}
// silu(x) = x / (1 + exp(-x)) (math.rs:82-84).
SYN_DEV float ref_silu(float x) { return x / (1.0f + ref_exp(-x)); }

// LDS written by some lanes of a wavefront, then read by others: order and complete the
// writes before the reads (single-wavefront code paths, where a workgroup barrier would not
// be reached by every wavefront).
SYN_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

SYN_DEV int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// a * b + c for operands of at most 24 significant bits (|a|, |b| < 2^23): one full-rate
// v_mad_i32_i24 instead of the quarter-rate 32-bit multiply.  Exact while the result fits 32 bits.
SYN_DEV int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

// The Q4_K super-block's exact S2 = sum_j m_j * s_j: 6-bit minimums m_j against the 32-value
// code sums s_j (|s_j| <= 32 * 128), every operand within 24 bits.  (S1 = sum_j sc_j * D_j takes
// mad24 the same way: |D_j| <= 32 * 15 * 128 < 2^16.)
SYN_DEV int q4k_s2(const int (&mn)[8], int4 sa, int4 sb) {
    int s2 = __mul24(mn[0], sa.x);
    s2 = mad24(mn[1], sa.y, s2);
    s2 = mad24(mn[2], sa.z, s2);
    s2 = mad24(mn[3], sa.w, s2);
    s2 = mad24(mn[4], sb.x, s2);
    s2 = mad24(mn[5], sb.y, s2);
    s2 = mad24(mn[6], sb.z, s2);
    return mad24(mn[7], sb.w, s2);
}

// Lane rotation by one inside groups of P lanes (the in-order fold hands its running sum to
// the next lane of the group): quad_perm [3,0,1,2], row_ror:1, or wave_ror:1.
template <int P>
SYN_DEV float rot1(float v) {
    int i = __builtin_bit_cast(int, v);
    if constexpr (P == 4) {
        i = __builtin_amdgcn_update_dpp(i, i, 0x93, 0xF, 0xF, false);
    } else if constexpr (P == 16) {
        i = __builtin_amdgcn_update_dpp(i, i, 0x121, 0xF, 0xF, false);
    } else {
        static_assert(P == 64, "P must be 4, 16 or 64");
        i = __builtin_amdgcn_update_dpp(i, i, 0x13C, 0xF, 0xF, false);
    }
    return __builtin_bit_cast(float, i);
}

// Reductions across lanes without LDS, for operations that are commutative and associative
// (max, sum, or): the quad steps pair lanes i ^ 1 and i ^ 2; then row_half_mirror pairs lane i
// of a group of eight with lane 7 - i (the other quad), row_mirror lane i of a row of 16 with
// lane 15 - i (the other half), and the permlane swaps rows 0-1 / 2-3, then the two halves of
// the wavefront.  Every lane of the group ends holding the group's result; every lane of the
// group must be active.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
template <int CTRL>
SYN_DEV uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}
// the maximum / minimum of 32-bit words over groups of G = 8, 16 or 64 lanes
template <int G, bool MIN>
SYN_DEV uint32_t group_ext_u32(uint32_t k) {
    auto op = [](uint32_t a, uint32_t b) { return MIN ? (a < b ? a : b) : (a > b ? a : b); };
    k = op(k, dpp_u32<DPP_XOR1>(k));
    k = op(k, dpp_u32<DPP_XOR2>(k));
    k = op(k, dpp_u32<DPP_HALF_MIRROR>(k));
    if constexpr (G >= 16) k = op(k, dpp_u32<DPP_MIRROR>(k));
    if constexpr (G == 64) {
        const auto s1 = __builtin_amdgcn_permlane16_swap(k, k, false, false);
        k = op(s1[0], s1[1]);
        const auto s2 = __builtin_amdgcn_permlane32_swap(k, k, false, false);
        k = op(s2[0], s2[1]);
    }
    return k;
}
template <int G>
SYN_DEV uint32_t group_max_u32(uint32_t k) { return group_ext_u32<G, false>(k); }
template <int G>
SYN_DEV uint32_t group_min_u32(uint32_t k) { return group_ext_u32<G, true>(k); }

// The signed maximum of a Q8_K block held N values a lane by G lanes (value i of the lane is the
// block's value G0 + i): the largest magnitude, the first index on equal magnitudes, and that
// value's sign.  Magnitudes compare as their bits (non-negative F32 patterns order as their
// values); `bad` is a NaN or an infinity anywhere in the block (its magnitude bits are the
// largest).  The first index is the smallest (index << 1 | sign) among the values of the
// largest magnitude.
template <int G, int N>
SYN_DEV void block_signed_amax(const float (&v)[N], int i0, float& amax, float& mx, bool& bad) {
    uint32_t mag[N], m = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        mag[i] = f2u(v[i]) & 0x7FFFFFFFu;
        m = m > mag[i] ? m : mag[i];
    }
    const uint32_t lm = m;  // the lane's own largest magnitude
    m = group_max_u32<G>(m);
    // the lane's first value of the largest magnitude (the scan runs backwards: the first wins);
    // lanes hold consecutive index ranges, so (i0 << 1 | its sign) orders as its (index << 1 | sign)
    uint32_t first = 0;
#pragma unroll
    for (int i = N - 1; i >= 0; --i) first = mag[i] == m ? f2u(v[i]) : first;
    uint32_t key = lm == m ? (((uint32_t)i0 << 1) | (first >> 31)) : 0xFFFFFFFFu;
    key = group_min_u32<G>(key);
    bad = m >= 0x7F800000u;
    amax = u2f(m);
    mx = (key & 1u) ? -amax : amax;
}

// the sum (or the or: OR = true) over groups of 8 lanes
template <bool OR = false>
SYN_DEV int group8_sum(int s) {
    auto op = [](int a, int b) { return OR ? (a | b) : a + b; };
    s = op(s, (int)dpp_u32<DPP_XOR1>((uint32_t)s));
    s = op(s, (int)dpp_u32<DPP_XOR2>((uint32_t)s));
    return op(s, (int)dpp_u32<DPP_HALF_MIRROR>((uint32_t)s));
}

// Q8_K of one 256-value block (crates/kernels-cpu/src/gemv/act.rs:351-373): largest
// magnitude, first index on ties, ggml's nearest_int; non-finite block -> scale NaN, codes 0.
// One wavefront; lane l holds values 4l..4l+3 and gets their four codes (packed bytes), the
// code sum of its 32-value sub-block l/8 (every lane of the sub-block) and the block scale.
struct Q8KLane {
    uint32_t packed;
    int sum32;
    float d;
};
SYN_DEV Q8KLane q8k_block_lane(float4 v4, int lane) {
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    // largest magnitude, the first index on a tie (an all-zero block gives amax 0)
    float amax, mx;
    bool bad;
    block_signed_amax<64>(v, lane * 4, amax, mx, bad);
    // codes of is v: is 0 where the codes are all 0 (an all-zero block, an infinite inverse
    // scale), which leaves finite values' codes 0; a block with a NaN or an infinity is zeroed
    // after the arithmetic (straight-line code)
    float d = 0.0f, is = 0.0f;
    if (bad) {
        d = __builtin_nanf("");
    } else if (amax != 0.0f) {
        const float iscale = neg127_div(mx);
        is = finite_f(iscale) ? iscale : 0.0f;  // |iscale v| <= 127 (to a rounding): nearest_int_small's range
        d = recip_rn(iscale);
    }
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = nearest_int_small(is * v[i]);
        q[i] = t < 127 ? t : 127;
    }
    Q8KLane r;
    r.packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
               ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    r.packed = bad ? 0u : r.packed;
    r.sum32 = group8_sum(sdot4(r.packed, 0x01010101u, 0));
    r.d = d;
    return r;
}
SYN_DEV Q8KLane q8k_block_lane(const float* __restrict__ xb, int lane) {
    return q8k_block_lane(reinterpret_cast<const float4*>(xb)[lane], lane);
}

// Q8_0 of one 32-value block (crates/kernels-cpu/src/gemv/act.rs:323-342): d = amax / 127,
// id = 1 / d, codes rounded to nearest even, the scale used the F16-rounded d; a non-finite
// block gets scale NaN and codes 0.  Eight lanes per block (every lane of the group of eight
// active): `sub` = lane & 7 holds values 4 sub .. 4 sub + 3 and gets their packed codes, the
// block's code sum and the scale.
struct Q8_0Lane {
    uint32_t packed;
    int sum;
    float d;
};
SYN_DEV Q8_0Lane q8_0_block_lane(float4 v4) {
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    // the largest magnitude by its bits (non-negative F32 patterns order as their values); a
    // NaN or an infinity has the largest bits, so the block is `bad` and its amax unused
    uint32_t ab = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = f2u(v[i]) & 0x7FFFFFFFu;
        ab = ab > a ? ab : a;
    }
    ab = group_max_u32<8>(ab);
    const bool bad = ab >= 0x7F800000u;
    const float amax = u2f(ab);
    // codes of is v, is 0 where the codes are all 0 (d 0, an infinite inverse); a bad block is
    // zeroed after the arithmetic (straight-line code)
    Q8_0Lane r;
    float is = 0.0f;
    if (bad) {
        r.d = __builtin_nanf("");
    } else {
        const float d = div127(amax);
        const float id = d != 0.0f ? recip_rn(d) : 0.0f;
        is = finite_f(id) ? id : 0.0f;
        r.d = f16_round(d);
    }
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = (int)__builtin_rintf(v[i] * is);
    r.packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) |
               ((uint32_t)(q[3] & 0xFF) << 24);
    r.packed = bad ? 0u : r.packed;
    r.sum = group8_sum(sdot4(r.packed, 0x01010101u, 0));
    return r;
}

// The same block in the row layout of the GEMV workspace: codes in order, the eight 32-value
// sums, the scale.
SYN_DEV void q8k_block_wave(const float* __restrict__ xb, int8_t* __restrict__ codes,
                            float* __restrict__ dout, int32_t* __restrict__ sums, int lane) {
    const Q8KLane r = q8k_block_lane(xb, lane);
    reinterpret_cast<uint32_t*>(codes)[lane] = r.packed;
    if ((lane & 7) == 0) sums[lane >> 3] = r.sum32;
    if (lane == 0) *dout = r.d;
}

// ---- LDS staging helpers of the matrix-core kernels ----------------------------------------

// s_waitcnt that waits for vector memory only: vmcnt n, expcnt and lgkmcnt left at their maxima.
template <int N>
SYN_DEV void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// The same for a wave-uniform n <= M.
template <int M>
SYN_DEV void wait_vm_n(int n) {
    if constexpr (M > 0) {
        if (n >= M) {
            wait_vm<M>();
            return;
        }
        wait_vm_n<M - 1>(n);
    } else {
        wait_vm<0>();
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// Workgroup barrier over LDS reads only: each wavefront's LDS reads have returned, then
// s_barrier.  (The fence of __syncthreads would also wait for every load into LDS still in
// flight, the next stages' included.)  The memory clobber keeps the compiler from moving
// memory accesses across it.
SYN_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The LDS address (M0 form) of a pointer into shared memory.
SYN_DEV uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lds_ptr)(p); }

// 16 bytes per active lane from sbase + voff to LDS address lds + 16 * lane, with no registers
// held while the load flies.  Written as assembly so the compiler does not track it (it would
// otherwise wait for every load into LDS in flight before each LDS read); the caller waits with
// wait_vm.  The LDS address is an m0 operand, so the compiler sets m0 itself; the s_nop covers
// the wait state between an SALU write of m0 and the LDS DMA.
SYN_DEV void lds_dma16(uint32_t voff, const void* sbase, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "{m0}"(lds)
                 : "memory");
}

// The rows a launch computes: `rows`, or fewer when `active` points at a step descriptor's
// rows_active (crates/kernels/include/syntropy/step_desc.h:53-57), read on the device so that a
// captured launch follows the value at each replay; `first` is the launch's first row.
SYN_DEV int active_rows(const uint32_t* active, int first, int rows) {
    if (!active) return rows;
    const int64_t a = (int64_t)*active - first;
    return a <= 0 ? 0 : (a < rows ? (int)a : rows);
}

// 4 bytes per active lane from sbase + voff to LDS address lds + 4 * lane (as lds_dma16).
SYN_DEV void lds_dma4(uint32_t voff, const void* sbase, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "{m0}"(lds)
                 : "memory");
}

}  // namespace syn
