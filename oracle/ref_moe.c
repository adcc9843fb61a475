/*
 * ref_moe.c -- TEST INFRASTRUCTURE ONLY: a driver around the reference's own split rule and
 * doorbell layout, crates/kernels/include/syntropy/moe_assign.h and moe_doorbell.h, compiled
 * from where they lie into oracle/_ref/libmoeref.so by `make -C oracle ref`.  Never shipped.
 *
 * ref_moe_assign       the header's syn_moe_assign, unchanged
 * ref_doorbell_layout  sizes, offsets and codes of the header's structs and macros
 * ref_moe_assign_compare
 *                      draws split-rule inputs and runs two rules on each (the header's and
 *                      the oracle's restatement, passed as function pointers), returning the
 *                      first input on which their codes differ
 */
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "syntropy/moe_assign.h"

void ref_moe_assign(const void* route, uint32_t n_route, const uint32_t* eligible,
                    uint32_t n_experts, uint32_t b_copy, uint64_t expert_bytes, uint32_t copy_slots,
                    uint32_t* out) {
    syn_moe_assign((const struct syn_route_slot*)route, n_route, eligible, n_experts, b_copy,
                   expert_bytes, copy_slots, out);
}

void ref_doorbell_layout(uint64_t* v) {
    v[0] = sizeof(struct syn_doorbell_header);
    v[1] = offsetof(struct syn_doorbell_header, seq);
    v[2] = offsetof(struct syn_doorbell_header, n_route);
    v[3] = offsetof(struct syn_doorbell_header, n_pred);
    v[4] = sizeof(struct syn_route_slot);
    v[5] = offsetof(struct syn_route_slot, expert);
    v[6] = offsetof(struct syn_route_slot, tokens);
    v[7] = offsetof(struct syn_route_slot, cache_slot);
    v[8] = SYN_DOORBELL_ROUTE_OFFSET();
    v[9] = SYN_DOORBELL_PRED_OFFSET(8);
    v[10] = SYN_DOORBELL_LAYER_SIZE(8, 16);
    v[11] = SYN_MOE_MISS;
    v[12] = SYN_MOE_HIT;
    v[13] = SYN_MOE_CPU;
    v[14] = SYN_MOE_DOORBELL_ABI_VERSION;
}

typedef void (*rule_fn)(const void*, uint32_t, const uint32_t*, uint32_t, uint32_t, uint64_t,
                        uint32_t, uint32_t*);

/* xorshift64* stream for the inputs */
static uint64_t rs;
static uint64_t draw(void) {
    rs ^= rs >> 12;
    rs ^= rs << 25;
    rs ^= rs >> 27;
    return rs * 0x2545F4914F6CDD1Dull;
}
static uint64_t pick(uint64_t n) { return draw() % n; }

/* Inputs in the regimes the reference's property test covers
 * (crates/kernels/src/moe/tests.rs:341-420): no experts, experts outside the bitmap, repeated
 * experts, token ties (most counts 0..3) and large counts, hits, misses and the cache slot just
 * below MISS, empty, full and random bitmaps, zero and maximal budgets, zero, small, huge and
 * budget-sized experts, no copy slots, a few, u32::MAX of them and up to the entry count.
 * Returns the first case whose codes differ, or -1; *copies counts rule a's COPY codes. */
int64_t ref_moe_assign_compare(uint64_t seed, uint64_t cases, void* rule_a, void* rule_b,
                               uint64_t* copies) {
    rule_fn a = (rule_fn)rule_a, b = (rule_fn)rule_b;
    static struct syn_route_slot route[320];
    static uint32_t words[2048];
    static uint32_t out_a[320], out_b[320];
    rs = seed | 1u;
    uint64_t copied = 0;
    for (uint64_t c = 0; c < cases; ++c) {
        uint32_t experts;
        switch (pick(4)) {
            case 0: experts = 0; break;
            case 1: experts = 1 + (uint32_t)pick(8); break;
            case 2: experts = 1 + (uint32_t)pick(300); break;
            default: experts = 1 + (uint32_t)pick(65536); break;
        }
        const uint32_t n = (uint32_t)(pick(32) == 0 ? pick(300) : pick(40));
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t e = (experts == 0 || pick(8) == 0) ? (uint32_t)pick(65536) : (uint32_t)pick(experts);
            if (i > 0 && pick(16) == 0) e = route[pick(i)].expert;
            const uint32_t t = pick(4) == 0 ? (uint32_t)pick(65536) : (uint32_t)pick(4);
            uint32_t slot;
            if (pick(2) == 0)
                slot = SYN_MOE_MISS;
            else if (pick(16) == 0)
                slot = SYN_MOE_MISS - 1u;
            else
                slot = (uint32_t)pick(1u << 20);
            route[i].expert = (uint16_t)e;
            route[i].tokens = (uint16_t)t;
            route[i].cache_slot = slot;
        }
        const uint32_t nw = (experts + 31u) / 32u, density = (uint32_t)pick(4);
        for (uint32_t w = 0; w < nw; ++w)
            words[w] = density == 0 ? 0u : density == 1 ? 0xFFFFFFFFu
                     : density == 2 ? (uint32_t)draw() : (uint32_t)(draw() & draw());
        uint32_t b_copy;
        switch (pick(4)) {
            case 0: b_copy = 0; break;
            case 1: b_copy = 0xFFFFFFFFu; break;
            case 2: b_copy = (uint32_t)pick(1u << 20); break;
            default: b_copy = (uint32_t)draw(); break;
        }
        uint64_t eb;
        switch (pick(5)) {
            case 0: eb = 0; break;
            case 1: eb = 1 + pick(1u << 16); break;
            case 2: eb = 1 + pick(1u << 24); break;
            case 3: eb = draw(); break;
            default: eb = b_copy; break;
        }
        uint32_t slots;
        switch (pick(4)) {
            case 0: slots = 0; break;
            case 1: slots = (uint32_t)pick(8); break;
            case 2: slots = 0xFFFFFFFFu; break;
            default: slots = (uint32_t)pick((uint64_t)n + 1); break;
        }
        memset(out_a, 0xA5, sizeof out_a);
        memset(out_b, 0x5A, sizeof out_b);
        a(route, n, words, experts, b_copy, eb, slots, out_a);
        b(route, n, words, experts, b_copy, eb, slots, out_b);
        if (memcmp(out_a, out_b, (size_t)n * 4) != 0) return (int64_t)c;
        for (uint32_t i = 0; i < n; ++i) copied += out_a[i] < SYN_MOE_CPU;
    }
    if (copies) *copies = copied;
    return -1;
}
