"""Independent pins of the oracle's MoE packing, routing and combine (CPU only).

The reference has code for the packing only (crates/kernels-cpu/src/moe.rs:431-457); MoeRoute
and MoeCombine exist as a specification (plan/rfcs/RFC-0042-quantization-and-numerical-fidelity.md
:232-233, crates/kernels/src/reference.rs:56-59) and one test helper for the combine
(crates/kernels-cpu/src/moe/tests.rs:541-556).  Each check below is computed without the oracle's
code path (a library sort, hand-derived bits, exact arithmetic, an F64 bound), and each comes with
planted mistakes, applied to a CPU copy of the oracle's output, that the same check must reject.
"""
import numpy as np
import pytest

from oracle import oracle as o

f32 = np.float32


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- packing: moe.rs:431-457 (counting sort, stable in slot order) ---------------------------
def library_pack(ids, n_experts):
    """Offsets from bincount + cumsum; slots from numpy's stable argsort of the expert ids."""
    flat = np.asarray(ids, dtype=np.int64).ravel()
    counts = np.bincount(flat, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    return offsets, np.argsort(flat, kind="stable").astype(np.uint32)


def brute_pack(ids, n_experts):
    """The definition spelled out: experts ascending, each expert's slots r*k+j in slot order."""
    flat = [int(v) for v in np.asarray(ids).ravel()]
    offsets, slots = [0], []
    for e in range(n_experts):
        slots += [s for s, v in enumerate(flat) if v == e]
        offsets.append(len(slots))
    return np.array(offsets, np.uint32), np.array(slots, np.uint32)


def pack_cases():
    rs = np.random.default_rng(0xAC4)
    cases = []
    for rows, k, e in [(1, 1, 1), (1, 8, 128), (5, 2, 6), (64, 8, 128), (37, 4, 16), (3, 3, 300)]:
        cases.append((np.stack([rs.permutation(e)[:k] for _ in range(rows)]).astype(np.int32), e))
    # skewed: three experts take most slots, most experts are empty
    ids = np.where(rs.random((96, 8)) < 0.7, rs.integers(0, 3, (96, 8)), rs.integers(0, 128, (96, 8)))
    cases.append((ids.astype(np.int32), 128))
    # every slot on one expert (repeats within a row are legal input to the packing)
    cases.append((np.full((9, 4), 5, np.int32), 8))
    cases.append((np.zeros((0, 8), np.int32), 128))
    return cases


def check_pack(fn, cases):
    for ids, e in cases:
        offsets, slots = fn(ids, e)
        want_o, want_s = library_pack(ids, e)
        if not (np.array_equal(offsets, want_o) and np.array_equal(slots, want_s)):
            return False
    return True


def test_pack_equals_a_library_stable_sort_and_brute_force():
    cases = pack_cases()
    assert check_pack(o.moe_pack, cases)
    for ids, e in cases:
        if ids.size <= 1024:
            bo, bs = brute_pack(ids, e)
            go, gs = o.moe_pack(ids, e)
            assert np.array_equal(go, bo) and np.array_equal(gs, bs)


def test_pack_at_the_prefill_shape():
    """2048 tokens x top-8 of 128 experts, with three experts over-loaded."""
    rs = np.random.default_rng(2048)
    hot = rs.random((2048, 8)) < 0.15
    ids = np.where(hot, rs.choice([3, 50, 97], (2048, 8)), rs.integers(0, 128, (2048, 8))).astype(np.int32)
    assert check_pack(o.moe_pack, [(ids, 128)])


def test_pack_catches_planted_mistakes():
    cases = pack_cases()

    def unstable(ids, e):  # each expert's slots in reverse slot order
        off, sl = o.moe_pack(ids, e)
        sl = sl.copy()
        for a in range(e):
            sl[off[a]:off[a + 1]] = sl[off[a]:off[a + 1]][::-1]
        return off, sl

    def inclusive(ids, e):  # offsets[e] left at the cursor (the end of expert e)
        off, sl = o.moe_pack(ids, e)
        return np.concatenate([off[1:], off[-1:]]), sl

    def row_not_slot(ids, e):  # the row index stored instead of the slot index
        off, sl = o.moe_pack(ids, e)
        return off, sl // max(ids.shape[1], 1)

    def descending(ids, e):  # experts walked from the highest id down
        return o.moe_pack((e - 1 - np.asarray(ids)).astype(np.int32), e)

    for bad in (unstable, inclusive, row_not_slot, descending):
        assert not check_pack(bad, cases), bad.__name__


def test_pack_refuses_ids_outside_the_experts():
    for bad in (-1, 16, 1 << 30):
        ids = np.array([[0, 3], [bad, 2]], np.int32)
        with pytest.raises(ValueError):
            o.moe_pack(ids, 16)


# ---- combine: moe/tests.rs:541-556 ---------------------------------------------------------
def combine_hand_cases():
    """(out [rows, k, hidden], ids, w, want [rows, hidden]) with the answer derived by hand."""
    cases = []
    # Expert order 1, 3, 5 sums 2^27 - 2^27 + 1 = 1; slot order would give (1 + 2^27) - 2^27 = 0
    # (2^27 + 1 rounds to 2^27) and descending order (1 - 2^27) + 2^27 = 0.
    out = np.array([[[1.0], [2.0 ** 27], [-(2.0 ** 27)]]], f32)
    cases.append((out, np.array([[5, 1, 3]], np.int32), np.ones((1, 3), f32), np.array([[1.0]], f32)))
    # Each product rounded before its add: expert 2 comes first, y = 1 * -1 = -1; expert 7 then
    # adds fl(a * a) = 1 + 2^-11 (the exact square 1 + 2^-11 + 2^-24 is a tie, to even), so
    # y = 2^-11; a fused multiply-add would keep the 2^-24 and give 2^-11 + 2^-24.
    a = f32(1 + 2.0 ** -12)
    out = np.array([[[a], [-1.0]]], f32)
    cases.append((out, np.array([[7, 2]], np.int32), np.array([[a, 1.0]], f32),
                  np.array([[2.0 ** -11]], f32)))
    return cases


def exact_case(seed, rows=13, k=8, hidden=64, n_experts=32):
    """Small integers times powers of two: every product and partial sum is exact, so the
    answer is the integer sum over the slots in any order."""
    rs = np.random.default_rng(seed)
    out = rs.integers(-1000, 1001, (rows, k, hidden)).astype(f32)
    w = (2.0 ** rs.integers(-3, 4, (rows, k))).astype(f32)
    ids = np.stack([rs.permutation(n_experts)[:k] for _ in range(rows)]).astype(np.int32)
    want = (out.astype(np.float64) * w[:, :, None]).sum(axis=1).astype(f32)
    return out, ids, w, want


def one_hot_case(seed, rows=11, k=8, hidden=40, n_experts=64):
    rs = np.random.default_rng(seed)
    out = rs.standard_normal((rows, k, hidden)).astype(f32)
    ids = np.stack([rs.permutation(n_experts)[:k] for _ in range(rows)]).astype(np.int32)
    hot = rs.integers(0, k, rows)
    w = np.zeros((rows, k), f32)
    w[np.arange(rows), hot] = 1.0
    return out, ids, w, out[np.arange(rows), hot]


def check_combine(fn):
    cases = combine_hand_cases() + [exact_case(s) for s in (1, 2)] + [one_hot_case(3)]
    return all(np.array_equal(bits(fn(out, ids, w)), bits(want)) for out, ids, w, want in cases)


def test_combine_matches_hand_exact_and_one_hot_cases():
    assert check_combine(o.moe_combine)


def test_combine_catches_planted_mistakes():
    def ordered(order_of, fused=False, by_rank=False):
        def fn(out, ids, w):
            rows, k, hidden = out.shape
            y = np.zeros((rows, hidden), f32)
            for r in range(rows):
                for a, j in enumerate(order_of(ids[r])):
                    wj = w[r, a] if by_rank else w[r, j]
                    if fused:
                        y[r] = (y[r].astype(np.float64) + np.float64(wj) * out[r, j]).astype(f32)
                    else:
                        y[r] = y[r] + f32(wj) * out[r, j]
            return y
        return fn

    ascending = lambda ids: np.argsort(ids, kind="stable")  # noqa: E731
    assert check_combine(ordered(ascending))  # the helper's definition itself passes
    assert not check_combine(ordered(lambda ids: range(len(ids))))  # slot order
    assert not check_combine(ordered(lambda ids: np.argsort(-ids, kind="stable")))  # descending
    assert not check_combine(ordered(ascending, fused=True))
    assert not check_combine(ordered(ascending, by_rank=True))


# ---- combine as the graph binds it: [per_expert, weights, shared...], rank order ---------------
# (crates/graph/src/ir/signature.rs:153, crates/graph/src/blocks/ffn.rs:189-200; RFC-0042 ...md:233)
def ranked_hand_cases():
    """(out [rows, k, hidden], w, shared list, want [rows, hidden]) derived by hand."""
    cases = []
    # Rank order 0, 1, 2 sums (2^27 + 1) - 2^27 = 0 (2^27 + 1 rounds to 2^27); ascending expert
    # order of ids [5, 1, 3] would give 1 (the helper's first hand case), reversed order 1 too.
    out = np.array([[[2.0 ** 27], [1.0], [-(2.0 ** 27)]]], f32)
    cases.append((out, np.ones((1, 3), f32), [], np.array([[0.0]], f32)))
    # Each product rounded before its add: rank 0 gives -1, rank 1 adds fl(a * a) = 1 + 2^-11,
    # y = 2^-11; a fused multiply-add would keep the 2^-24.
    a = f32(1 + 2.0 ** -12)
    out = np.array([[[-1.0], [a]]], f32)
    cases.append((out, np.array([[1.0, a]], f32), [], np.array([[2.0 ** -11]], f32)))
    # The shared outputs come after the routed slots and carry no weight: the slot gives
    # 4 * 2^25 = 2^27, then each shared 8 is half an ulp of 2^27 (a tie, to even: lost), y = 2^27;
    # shared first would give 8 + 8 = 16, then 2^27 + 16 exactly; weighting them by 4 would give
    # 2^27 + 32 + 32.
    out = np.array([[[2.0 ** 25]]], f32)
    cases.append((out, np.array([[4.0]], f32), [np.array([[8.0]], f32), np.array([[8.0]], f32)],
                  np.array([[2.0 ** 27]], f32)))
    return cases


def ranked_exact_case(seed, rows=13, k=8, hidden=64, n_shared=2):
    rs = np.random.default_rng(seed)
    out = rs.integers(-1000, 1001, (rows, k, hidden)).astype(f32)
    w = (2.0 ** rs.integers(-3, 4, (rows, k))).astype(f32)
    shared = [rs.integers(-1000, 1001, (rows, hidden)).astype(f32) for _ in range(n_shared)]
    want = (out.astype(np.float64) * w[:, :, None]).sum(axis=1) + sum(a.astype(np.float64) for a in shared)
    return out, w, shared, want.astype(f32)


def check_ranked(fn):
    cases = ranked_hand_cases() + [ranked_exact_case(s) for s in (4, 5)]
    ok = all(np.array_equal(bits(fn(out, w, sh)), bits(want)) for out, w, sh, want in cases)
    # rows whose ids ascend: the rank-order sum is the helper's ascending-expert sum
    rs = np.random.default_rng(6)
    out = rs.standard_normal((9, 8, 48)).astype(f32)
    w = rs.random((9, 8)).astype(f32)
    ids = np.sort(np.stack([rs.permutation(128)[:8] for _ in range(9)]), axis=1).astype(np.int32)
    return ok and np.array_equal(bits(fn(out, w, [])), bits(o.moe_combine(out, ids, w)))


def test_combine_ranked_matches_hand_exact_and_ascending_cases():
    assert check_ranked(o.moe_combine_ranked)


def test_combine_ranked_catches_planted_mistakes():
    def variant(order=lambda k: range(k), fused=False, shared_first=False, shared_weight=1.0):
        def fn(out, w, shared):
            rows, k, hidden = out.shape
            y = np.zeros((rows, hidden), f32)
            for r in range(rows):
                def routed():
                    for j in order(k):
                        if fused:
                            y[r] = (y[r].astype(np.float64) + np.float64(w[r, j]) * out[r, j]).astype(f32)
                        else:
                            y[r] = y[r] + f32(w[r, j]) * out[r, j]

                def sh():
                    for a in shared:
                        y[r] = y[r] + f32(shared_weight) * a[r]
                if shared_first:
                    sh()
                    routed()
                else:
                    routed()
                    sh()
            return y
        return fn

    assert check_ranked(variant())  # the definition itself passes
    assert not check_ranked(variant(order=lambda k: reversed(range(k))))
    assert not check_ranked(variant(fused=True))
    assert not check_ranked(variant(shared_first=True))
    assert not check_ranked(variant(shared_weight=4.0))


# ---- MoeRoute{Softmax}: RFC-0042 ...md:232-233; reference.rs:56-59 -----------------------------
def route_logits(logits):
    """A router and a one-hot token that make the F32Fixed logits exactly `logits`."""
    e = len(logits)
    router = np.zeros((e, 32), f32)
    router[:, 0] = logits
    x = np.zeros((1, 32), f32)
    x[0, 0] = 1.0
    return router, x


def hand_route(logits, top_k, reciprocal=False, subtract_max=True):
    """The specification evaluated step by step in F32: m = max, e_i = exp(l_i - m) with the
    reference's software exp, s = the sum in index order (one 32-value block), p_i = e_i / s;
    ids by (p descending, index ascending); w = p_sel / (sum of p_sel in rank order)."""
    l = np.asarray(logits, f32)
    m = l.max() if subtract_max else f32(0)
    e = np.array([o.exp(float(f32(v - m))) for v in l], f32)
    s = f32(0)
    for v in e:
        s = f32(s + v)
    p = (e * (f32(1) / s)).astype(f32) if reciprocal else (e / s).astype(f32)
    ids = np.lexsort((np.arange(len(l)), -p))[:top_k]
    sel = p[ids]
    t = f32(0)
    for v in sel:
        t = f32(t + v)
    w = (sel * (f32(1) / t)).astype(f32) if reciprocal else (sel / t).astype(f32)
    return ids.astype(np.int32), w, p


@pytest.mark.parametrize("logits,top_k", [
    ([0, -1, -3, 0.5], 3),  # division and renormalization both differ from reciprocal multiplies
    ([0, -1, 0, -2], 3),  # a tie between experts 0 and 2: the lower index ranks first
    ([100, 99.5, 98, 0], 2),  # exp(100) overflows: only the max-subtracted form is finite
    ([-200, -1, -150, 0, -1], 4),  # exp of -200 - 0 underflows to +0; ties at -1
])
def test_route_hand_cases(logits, top_k):
    router, x = route_logits(logits)
    ids, w, p = o.moe_route(router, x, len(logits), top_k)
    hid, hw, hp = hand_route(logits, top_k)
    assert (ids[0] == hid).all()
    assert np.array_equal(bits(p[0]), bits(hp))
    assert np.array_equal(bits(w[0]), bits(hw))


def test_route_hand_cases_reject_planted_mistakes():
    """The reciprocal-multiply and no-max-subtract variants give other bits on the cases above."""
    ids, w, p = hand_route([0, -1, -3, 0.5], 3)
    rid, rw, rp = hand_route([0, -1, -3, 0.5], 3, reciprocal=True)
    assert not np.array_equal(bits(p), bits(rp)) and not np.array_equal(bits(w), bits(rw))
    _, nw, npr = hand_route([100, 99.5, 98, 0], 2, subtract_max=False)
    assert np.isnan(npr[:3]).all() and np.isnan(nw).all()  # inf / inf
    ids, _, p = hand_route([0, -1, 0, -2], 3)
    assert ids.tolist() == [0, 2, 1] and p[0] == p[2]


def route_bound(logits_row, n):
    """Relative error bound of each probability against the F64 softmax of the same F32 logits:
    the subtraction (|l - m| 2^-24 in exp's argument), exp (2 ulp), the same for every term of
    the sum plus its (31 + tree levels) roundings, and the division."""
    span = float(np.max(np.abs(logits_row - logits_row.max())))
    levels = max(0, int(np.ceil(np.log2(max(1, -(-n // 32))))))
    return (2 * (span * 2 ** -24 + 2 * 2 ** -23) + (31 + levels) * 2 ** -24 + 2 ** -24) * 1.01


def route_inputs(seed, rows, hidden, n_experts, scale=1.0):
    router = o.normal(seed, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    x = o.normal(seed + 1, 1.0, rows * hidden).reshape(rows, hidden) * f32(scale)
    return router, x.astype(f32)


@pytest.mark.parametrize("rows,hidden,n_experts,top_k,scale", [
    (64, 4096, 128, 8, 1.0), (16, 512, 60, 6, 1.0), (8, 256, 256, 8, 1.0),
    (8, 4096, 128, 8, 8.0),  # logit spans near 70: the max subtraction matters
])
def test_route_probabilities_within_the_f64_bound(rows, hidden, n_experts, top_k, scale):
    router, x = route_inputs(0x51A3 + rows, rows, hidden, n_experts, scale)
    ids, w, p = o.moe_route(router, x, n_experts, top_k)
    logits = np.array([[o.fdot(router[e], x[r]) for e in range(n_experts)] for r in range(rows)], f32)
    for r in range(rows):
        l64 = logits[r].astype(np.float64)
        e64 = np.exp(l64 - l64.max())
        p64 = e64 / e64.sum()
        rel = np.abs(p[r] - p64) / p64
        assert (rel <= route_bound(logits[r], n_experts)).all(), (r, rel.max())
        assert abs(float(p[r].astype(np.float64).sum()) - 1.0) <= 64 * 2 ** -24
        # ids: a library sort of the probabilities by (p descending, index ascending)
        assert (ids[r] == np.lexsort((np.arange(n_experts), -p[r]))[:top_k]).all()
        # renormalized weights sum to 1 within k + 1 roundings, keep the ranking and the ratios
        assert abs(float(w[r].astype(np.float64).sum()) - 1.0) <= (top_k + 2) * 2 ** -24
        assert (np.diff(w[r]) <= 0).all()
        ratio = (p[r, ids[r]].astype(np.float64) / p[r, ids[r]].astype(np.float64).sum())
        assert np.allclose(w[r], ratio, rtol=(top_k + 3) * 2 ** -24, atol=0)
    _, w_plain, p_plain = o.moe_route(router, x, n_experts, top_k, renormalize=False)
    assert np.array_equal(bits(w_plain), bits(np.take_along_axis(p_plain, ids, axis=1)))


def test_route_bound_rejects_a_dropped_term():
    """A softmax whose sum skips the last expert misses the bound (the check is not vacuous)."""
    router, x = route_inputs(0x51A3, 4, 4096, 128)
    logits = np.array([o.fdot(router[e], x[0]) for e in range(128)], f32)
    l64 = logits.astype(np.float64)
    e64 = np.exp(l64 - l64.max())
    p64 = e64 / e64.sum()
    e32 = np.array([o.exp(float(f32(v - logits.max()))) for v in logits], f32)
    wrong = (e32 / f32(o.fsum(e32[:-1]))).astype(f32)
    assert (np.abs(wrong - p64) / p64 > route_bound(logits, 128)).any()
