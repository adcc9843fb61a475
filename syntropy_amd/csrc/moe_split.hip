// The MoE residency split on gfx950: the router's doorbell layer and the split rule that every
// site evaluates from it (HIT / COPY / CPU per routed expert).
//
//  * doorbell: crates/kernels/include/syntropy/moe_doorbell.h (layout, little-endian) and
//    plan/rfcs/RFC-0040-kernel-providers-and-backends.md:390 (contents): the step's seq (the low
//    32 bits of syn_step_desc.step), then one syn_route_slot { expert, tokens, cache_slot } per
//    distinct expert the pass selected, tokens the rows that selected it, cache_slot the
//    expert's slot_of entry.  Entries are in ascending expert index; n_pred is 0.
//  * split rule: crates/kernels/include/syntropy/moe_assign.h:29-61, bit-identical: a hit is
//    HIT; an eligible miss takes copy slot c, its rank among the eligible misses in the order
//    (tokens descending, expert ascending, entry ascending), while c < copy_slots and
//    (c + 1) * expert_bytes <= b_copy; every other miss is CPU.
//
// One lane per route entry, as the reference's GPU version (kernels-metal/shaders/
// moe_assign.metal:130-143); the rank is a count over every entry, so each workgroup stages the
// entries' order keys through LDS in tiles and every lane compares its key with the whole tile
// (LDS broadcast reads).  The doorbell is one workgroup: a per-expert histogram in LDS, then a
// scan that compacts the selected experts in ascending order.
#include "common.hpp"
#include "kernels.hpp"

namespace syn {

namespace {

constexpr uint32_t MOE_MISS = 0xFFFFFFFFu;
constexpr uint32_t MOE_HIT = 0xFFFFFFFFu;
constexpr uint32_t MOE_CPU = 0xFFFFFFFEu;
constexpr int AS_THREADS = 256;
constexpr int AS_TILE = 1024;

// One syn_route_slot read as two words: expert | tokens << 16, cache_slot.
SYN_DEV uint2 route_at(const uint8_t* route, uint32_t i) {
    return *reinterpret_cast<const uint2*>(route + 8ull * i);
}

SYN_DEV bool eligible_miss(uint2 r, const uint32_t* eligible, uint32_t n_experts) {
    const uint32_t e = r.x & 0xFFFFu;
    return r.y == MOE_MISS && e < n_experts && ((eligible[e >> 5] >> (e & 31u)) & 1u);
}

// The walk order of the eligible misses as one u64: tokens descending, then expert, then entry.
SYN_DEV uint64_t order_key(uint2 r, uint32_t i) {
    const uint64_t tokens = r.x >> 16, expert = r.x & 0xFFFFu;
    return ((0xFFFFull - tokens) << 48) | (expert << 32) | i;
}

}  // namespace

// LAYER = 1: route and n_route come from a doorbell layer (its header's n_route, checked against
// max_union) and b_copy from a device word; LAYER = 0: a route array and host values.
template <int LAYER>
__global__ __launch_bounds__(AS_THREADS) void k_moe_assign(const uint8_t* __restrict__ src, uint32_t n_route,
                                                           uint32_t max_union,
                                                           const uint32_t* __restrict__ eligible,
                                                           uint32_t n_experts,
                                                           const uint32_t* __restrict__ b_copy_at,
                                                           uint32_t b_copy, uint64_t expert_bytes,
                                                           uint32_t copy_slots, uint32_t* __restrict__ out) {
    __shared__ uint64_t keys[AS_TILE];
    const uint8_t* route = src;
    if (LAYER) {
        n_route = *reinterpret_cast<const uint16_t*>(src + 4);
        if (n_route > max_union) return;  // a layer the reader refuses: no codes
        b_copy = *b_copy_at;
        route = src + 8;
    }
    const uint32_t base = blockIdx.x * AS_THREADS;
    if (base >= n_route) return;  // uniform per workgroup
    const uint32_t i = base + threadIdx.x;
    const bool live = i < n_route;
    const uint2 r = live ? route_at(route, i) : make_uint2(0u, 0u);
    const bool em = live && eligible_miss(r, eligible, n_experts);
    const uint64_t key = order_key(r, i);
    uint32_t c = 0;
    for (uint32_t t0 = 0; t0 < n_route; t0 += AS_TILE) {
        __syncthreads();
        for (uint32_t q = threadIdx.x; q < AS_TILE; q += AS_THREADS) {
            const uint32_t j = t0 + q;
            uint64_t k = ~0ull;  // above every key: never counted
            if (j < n_route) {
                const uint2 rj = route_at(route, j);
                if (eligible_miss(rj, eligible, n_experts)) k = order_key(rj, j);
            }
            keys[q] = k;
        }
        __syncthreads();
        if (em) {
            const uint32_t m = n_route - t0 < (uint32_t)AS_TILE ? n_route - t0 : (uint32_t)AS_TILE;
            for (uint32_t q = 0; q < m; ++q) c += keys[q] < key;
        }
    }
    if (!live) return;
    uint32_t code;
    if (r.y != MOE_MISS)
        code = MOE_HIT;
    else if (em)
        code = (c < copy_slots && expert_bytes <= (uint64_t)b_copy && ((uint64_t)c + 1u) * expert_bytes <= (uint64_t)b_copy)
                   ? c
                   : MOE_CPU;
    else
        code = MOE_CPU;
    out[i] = code;
}

void launch_moe_assign(const uint8_t* route, uint32_t n_route, const uint32_t* eligible, uint32_t n_experts,
                       uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots, uint32_t* out,
                       hipStream_t stream) {
    if (n_route == 0) return;
    const dim3 grid((n_route + AS_THREADS - 1) / AS_THREADS);
    hipLaunchKernelGGL(k_moe_assign<0>, grid, dim3(AS_THREADS), 0, stream, route, n_route, 0u, eligible,
                       n_experts, nullptr, b_copy, expert_bytes, copy_slots, out);
}

void launch_moe_assign_layer(const uint8_t* layer, uint32_t max_union, const uint32_t* eligible,
                             uint32_t n_experts, const uint32_t* b_copy, uint64_t expert_bytes,
                             uint32_t copy_slots, uint32_t* out, hipStream_t stream) {
    if (max_union == 0) return;
    const dim3 grid((max_union + AS_THREADS - 1) / AS_THREADS);
    hipLaunchKernelGGL(k_moe_assign<1>, grid, dim3(AS_THREADS), 0, stream, layer, 0u, max_union, eligible,
                       n_experts, b_copy, 0u, expert_bytes, copy_slots, out);
}

// ============================================================================================
// The doorbell layer
// ============================================================================================

// One workgroup.  desc (optional): the step descriptor, whose step (offset 0) gives seq and
// whose rows_active (offset 8) bounds the rows.  status: 0, 1 for an id outside [0, n_experts),
// 2 when the distinct experts exceed max_union; the layer is written only with status 0.
__global__ __launch_bounds__(1024) void k_moe_doorbell(const int32_t* __restrict__ ids, int rows, int top_k,
                                                       int n_experts, const uint32_t* __restrict__ slot_of,
                                                       const uint32_t* __restrict__ desc, uint32_t seq,
                                                       uint8_t* __restrict__ layer, uint32_t max_union,
                                                       uint32_t* __restrict__ status) {
    extern __shared__ uint32_t cnt[];  // [n_experts]
    __shared__ uint32_t bad;
    __shared__ uint32_t wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (desc) {
        seq = desc[0];
        rows = active_rows(desc + 2, 0, rows);
    }
    for (int e = tid; e < n_experts; e += 1024) cnt[e] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    const int n = rows * top_k;
    for (int s = tid; s < n; s += 1024) {
        const int r = s / top_k, j = s - r * top_k;
        const int e = ids[s];
        if (e < 0 || e >= n_experts) {
            atomicOr(&bad, 1u);
            continue;
        }
        bool again = false;  // a row counts once per expert
        for (int q = 0; q < j; ++q) again |= ids[r * top_k + q] == e;
        if (!again) atomicAdd(&cnt[e], 1u);
    }
    __syncthreads();
    if (bad) {
        if (tid == 0 && status) status[0] = 1u;
        return;
    }
    // each thread owns `per` consecutive experts; an exclusive scan of their selected counts
    const int per = (n_experts + 1023) / 1024;
    const int e0 = tid * per;
    const int e1 = e0 + per < n_experts ? e0 + per : n_experts;
    uint32_t mine = 0;
    for (int e = e0; e < e1; ++e) mine += cnt[e] != 0u;
    uint32_t incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int w = 0; w < 16; ++w) {
        const uint32_t v = wsum[w];
        before += w < wave ? v : 0u;
        total += v;
    }
    if (total > max_union) {  // uniform
        if (tid == 0 && status) status[0] = 2u;
        return;
    }
    uint32_t at = before + incl - mine;
    uint2* route = reinterpret_cast<uint2*>(layer + 8);
    for (int e = e0; e < e1; ++e) {
        const uint32_t t = cnt[e];
        if (!t) continue;
        route[at++] = make_uint2((uint32_t)e | (t << 16), slot_of ? slot_of[e] : MOE_MISS);
    }
    if (tid == 0) {
        *reinterpret_cast<uint2*>(layer) = make_uint2(seq, total);  // n_route, n_pred = 0
        if (status) status[0] = 0u;
    }
}

size_t moe_doorbell_lds(int n_experts) { return sizeof(uint32_t) * (size_t)n_experts; }

void launch_moe_doorbell(const int32_t* ids, int rows, int top_k, int n_experts, const uint32_t* slot_of,
                         const void* desc, uint32_t seq, uint8_t* layer, uint32_t max_union, uint32_t* status,
                         hipStream_t stream) {
    hipLaunchKernelGGL(k_moe_doorbell, dim3(1), dim3(1024), moe_doorbell_lds(n_experts), stream, ids, rows, top_k,
                       n_experts, slot_of, (const uint32_t*)desc, seq, layer, max_union, status);
}

// ============================================================================================
// Site masks from the codes
// ============================================================================================

// site[e] = 1 for the experts of the layer's route whose code is of class `which` (0 HIT,
// 1 COPY, 2 CPU), 0 for every other expert: the mask MoeGrouped's site input takes.
__global__ __launch_bounds__(256) void k_moe_site_mask(const uint8_t* __restrict__ layer, uint32_t max_union,
                                                       const uint32_t* __restrict__ codes, int n_experts,
                                                       int which, int32_t* __restrict__ site) {
    const uint32_t n_route = *reinterpret_cast<const uint16_t*>(layer + 4);
    const bool ok = n_route <= max_union;
    for (int e = threadIdx.x; e < n_experts; e += 256) site[e] = 0;
    __syncthreads();
    if (!ok) return;
    const uint8_t* route = layer + 8;
    for (uint32_t i = threadIdx.x; i < n_route; i += 256) {
        const uint2 r = route_at(route, i);
        const uint32_t e = r.x & 0xFFFFu, c = codes[i];
        const int cls = c == MOE_HIT ? 0 : c == MOE_CPU ? 2 : 1;
        if (cls == which && e < (uint32_t)n_experts) site[e] = 1;
    }
}

void launch_moe_site_mask(const uint8_t* layer, uint32_t max_union, const uint32_t* codes, int n_experts,
                          int which, int32_t* site, hipStream_t stream) {
    hipLaunchKernelGGL(k_moe_site_mask, dim3(1), dim3(256), 0, stream, layer, max_union, codes, n_experts, which,
                       site);
}

}  // namespace syn
