"""Pins of the oracle's residency split (the split rule and the doorbell layer) against the
reference's own headers, compiled into oracle/_ref from crates/kernels/include/syntropy, and its
hand-worked tests (crates/kernels/src/moe/tests.rs).  CPU only."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as o

HIT, CPU, MISS = o.MOE_HIT, o.MOE_CPU, o.MOE_MISS


def need_ref():
    R = o.moe_ref_lib()
    if R is None:
        pytest.skip("oracle/_ref/libmoeref.so is not built (the reference tree is absent)")
    return R


def codes(entries, words, experts, b_copy, expert_bytes, copy_slots):
    return o.moe_assign(o.route_slots(entries), words, experts, b_copy, expert_bytes, copy_slots).tolist()


# ---- the split rule -----------------------------------------------------------------------
def test_split_rule_equals_the_reference_header_on_a_million_inputs():
    """The restatement of RFC-0040 3.4's walk equals the reference's generated C rule
    (moe_assign.h) on 10^6 drawn inputs, as moe/tests.rs:546-560 and :728-790 check theirs; the
    inputs reach the copy path."""
    R = need_ref()
    ref_fn = C.cast(R.ref_moe_assign, C.c_void_p).value
    or_fn = C.cast(o.lib().or_moe_assign, C.c_void_p).value
    copies = C.c_uint64(0)
    first = R.ref_moe_assign_compare(0x05EED0E17006, 1_000_000, ref_fn, or_fn, C.byref(copies))
    assert first == -1, f"case {first} differs"
    assert copies.value > 100_000


def test_split_rule_catches_a_planted_mistake():
    """The comparison fails for a rule that walks ties in the wrong order (expert descending):
    the drawn inputs are dense enough in ties to see it."""
    R = need_ref()
    proto = C.CFUNCTYPE(None, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64,
                        C.c_uint32, C.c_void_p)

    def wrong(route, n, words, experts, b_copy, eb, slots, out):
        r = np.ctypeslib.as_array(C.cast(route, C.POINTER(C.c_uint8)), (max(n, 1) * 8,))[: n * 8]
        rs = r.view(o.ROUTE_SLOT).copy()
        w = (np.ctypeslib.as_array(C.cast(words, C.POINTER(C.c_uint32)), ((experts + 31) // 32,)).copy()
             if experts else None)
        got = o.moe_assign(rs[::-1], w, experts, b_copy, eb, slots)[::-1]  # later entries first on ties
        C.memmove(out, got.ctypes.data, 4 * n)

    fn = proto(wrong)
    ref_fn = C.cast(R.ref_moe_assign, C.c_void_p).value
    first = R.ref_moe_assign_compare(7, 20_000, ref_fn, C.cast(fn, C.c_void_p).value, None)
    assert first >= 0


def test_worked_example():
    """moe/tests.rs:801-822: misses 7 (3 tokens), 2 (1), 5 (3), 9 (1, not eligible), a hit on 4."""
    route = [(7, 3, MISS), (4, 2, 11), (2, 1, MISS), (5, 3, MISS), (9, 1, MISS)]
    words = [1 << 2 | 1 << 5 | 1 << 7]
    assert codes(route, words, 16, 200, 100, 8) == [1, HIT, CPU, 0, CPU]
    assert codes(route, words, 16, 300, 100, 8) == [1, HIT, 2, 0, CPU]
    assert codes(route, words, 16, 300, 100, 1) == [CPU, HIT, CPU, 0, CPU]


def test_ties_go_to_the_lower_expert_then_the_earlier_entry():
    """moe/tests.rs:824-842."""
    allw = [0xFFFFFFFF]
    assert codes([(9, 2, MISS), (3, 2, MISS), (6, 2, MISS)], allw, 32, 0xFFFFFFFF, 1, 2) == [CPU, 0, 1]
    assert codes([(4, 1, MISS)] * 3, allw, 32, 0xFFFFFFFF, 1, 2) == [0, 1, CPU]


def test_zero_experts_and_outside_the_bitmap():
    """moe/tests.rs:844-872."""
    assert codes([], None, 0, 100, 1, 4) == []
    assert codes([(0, 1, MISS), (1, 1, 3)], None, 0, 0xFFFFFFFF, 1, 4) == [CPU, HIT]
    got = codes([(e, 1, MISS) for e in range(10)], [0xFFFFFFFF], 4, 0xFFFFFFFF, 1, 0xFFFFFFFF)
    assert got == [e if e < 4 else CPU for e in range(10)]
    assert codes([(65535, 1, MISS)], [0xFFFFFFFF], 4, 0xFFFFFFFF, 1, 1) == [CPU]


def test_budgets_at_their_limits():
    """moe/tests.rs:874-902."""
    allw = [0xFFFFFFFF] * 2
    route = [(e, 1, MISS) for e in range(40)]

    def copies(b, eb, slots):
        return sum(c < CPU for c in codes(route, allw, 64, b, eb, slots))

    assert copies(0xFFFFFFFF, 2**64 - 1, 0xFFFFFFFF) == 0
    assert copies(0xFFFFFFFF, 2**32, 9) == 0
    assert copies(0xFFFFFFFF, 2**32 - 1, 9) == 1
    assert copies(0, 0, 7) == 7
    assert copies(0xFFFFFFFF, 1, 0) == 0
    assert copies(0, 1, 9) == 0


def test_largest_doorbell():
    """moe/tests.rs:904-924: 65535 entries, all hits, then all misses with none eligible."""
    n = 65535
    hits = np.zeros(n, o.ROUTE_SLOT)
    hits["expert"] = np.arange(n)
    hits["tokens"] = 1
    hits["cache_slot"] = np.arange(n)
    assert (o.moe_assign(hits, None, 0, 0xFFFFFFFF, 1, 0xFFFFFFFF) == HIT).all()
    misses = hits.copy()
    misses["cache_slot"] = MISS
    assert (o.moe_assign(misses, np.zeros(2048, np.uint32), 65536, 0xFFFFFFFF, 1, 0xFFFFFFFF) == CPU).all()


def test_entry_order_does_not_change_the_decisions():
    """moe/tests.rs:612-627: for distinct experts, permuting the doorbell permutes the codes."""
    rs = np.random.default_rng(3)
    for _ in range(200):
        n = int(rs.integers(0, 48))
        route = np.zeros(n, o.ROUTE_SLOT)
        route["expert"] = rs.permutation(48)[:n]
        route["tokens"] = rs.integers(0, 4, n)
        route["cache_slot"] = np.where(rs.random(n) < 0.5, MISS, rs.integers(0, 64, n))
        words = rs.integers(0, 2**32, 2, dtype=np.uint64).astype(np.uint32)
        args = (words, 48, int(rs.integers(0, 40)), int(rs.integers(0, 6)), int(rs.integers(0, 12)))
        a = o.moe_assign(route, *args)
        perm = rs.permutation(n)
        b = o.moe_assign(route[perm], *args)
        assert (b == a[perm]).all()


# ---- the doorbell layer ---------------------------------------------------------------------
def test_doorbell_layout_matches_the_reference_header():
    """Struct sizes, offsets, macros and codes of moe_doorbell.h, as compiled; and
    moe/tests.rs:931-939 by hand (MAX_UNION 8, MAX_PRED 16: 8, 72, 200)."""
    R = need_ref()
    v = (C.c_uint64 * 15)()
    R.ref_doorbell_layout(v)
    assert list(v) == [8, 0, 4, 6, 8, 0, 2, 4, 8, 72, 200, MISS, HIT, CPU, 1]
    assert o.ROUTE_SLOT.itemsize == 8 and o.ROUTE_SLOT.fields["cache_slot"][1] == 4


def test_doorbell_bytes_by_hand():
    """The header and route bytes of moe/tests.rs:941-961's example, written from ids: seq
    0xDEADBEEF, expert 3 selected by two rows, a miss; then expert 5 in a cache slot."""
    ids = np.array([[3], [3], [5]], np.int32)
    slot_of = np.full(8, MISS, np.uint32)
    slot_of[5] = 0x01020304
    layer = o.moe_doorbell(ids, 8, 4, slot_of, seq=0xDEADBEEF)
    assert layer[:24].tolist() == [0xEF, 0xBE, 0xAD, 0xDE, 2, 0, 0, 0,
                                   3, 0, 2, 0, 255, 255, 255, 255,
                                   5, 0, 1, 0, 4, 3, 2, 1]
    assert (layer[24:] == 0).all()


def brute_doorbell(ids, n_experts, slot_of):
    tokens = {}
    for row in ids:
        for e in set(int(v) for v in row):
            tokens[e] = tokens.get(e, 0) + 1
    return [(e, tokens[e], MISS if slot_of is None else int(slot_of[e])) for e in sorted(tokens)]


def test_doorbell_route_list_against_a_brute_force_count():
    rs = np.random.default_rng(5)
    for rows, top_k, E in [(1, 1, 4), (7, 2, 16), (64, 8, 128), (300, 4, 256), (5, 3, 3), (40, 6, 8192)]:
        ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
        if rows > 3:
            ids[2, -1] = ids[2, 0]  # a row naming an expert twice counts it once
        slot_of = np.where(rs.random(E) < 0.5, MISS, rs.integers(0, 1 << 20, E)).astype(np.uint32)
        want = brute_doorbell(ids, E, slot_of)
        layer = o.moe_doorbell(ids, E, len(want), slot_of, seq=rows)
        n = int(layer[4:6].view(np.uint16)[0])
        assert int(layer[:4].view(np.uint32)[0]) == rows and n == len(want)
        assert int(layer[6:8].view(np.uint16)[0]) == 0
        got = layer[8:8 + 8 * n].view(o.ROUTE_SLOT)
        assert [tuple(int(x) for x in g) for g in got] == want
        assert o.moe_doorbell(ids, E, len(want) - 1, slot_of) is None  # too many routes


def test_doorbell_refuses_bad_ids():
    assert o.moe_doorbell(np.array([[0, 4]], np.int32), 4, 8) is None
    assert o.moe_doorbell(np.array([[-1, 2]], np.int32), 4, 8) is None
