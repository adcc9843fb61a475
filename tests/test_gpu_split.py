"""GPU parity of the MoE residency split against the oracle: the doorbell layer the router's ids
produce, the split rule's codes (bit-exact, on drawn inputs and the reference's hand-worked
cases), the codes read from a doorbell on the device, a captured graph that follows the step
descriptor, and the three sites' MoeGrouped launches completing one layer."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o

pytestmark = pytest.mark.gpu

HIT, CPU, MISS = o.MOE_HIT, o.MOE_CPU, o.MOE_MISS
SENTINEL = 0x7FC0DEAD


@pytest.fixture(scope="module")
def M():
    require_gpu()
    import syntropy_amd.moe as M
    return M


def gpu_codes(M, route, words, experts, b_copy, eb, slots):
    n = len(route)
    if n == 0:
        return []
    out = torch.full((n + 4,), 0x3A3A3A3A, dtype=torch.int32, device="cuda")
    M.assign(dev(route.view(np.uint8)), n, dev(words) if experts else None, experts, b_copy, eb, slots,
             out=out)
    got = host(out).view(np.uint32)
    assert (got[n:] == 0x3A3A3A3A).all(), "a code past the route was written"
    return got[:n].tolist()


def draw_case(rs):
    """Split-rule inputs in the regimes of crates/kernels/src/moe/tests.rs:341-420."""
    experts = [0, int(rs.integers(1, 9)), int(rs.integers(1, 301)), int(rs.integers(1, 65537))][rs.integers(4)]
    n = int(rs.integers(0, 300)) if rs.integers(32) == 0 else int(rs.integers(0, 40))
    route = np.zeros(n, o.ROUTE_SLOT)
    for i in range(n):
        e = int(rs.integers(65536)) if (experts == 0 or rs.integers(8) == 0) else int(rs.integers(experts))
        if i > 0 and rs.integers(16) == 0:
            e = int(route["expert"][rs.integers(i)])
        t = int(rs.integers(65536)) if rs.integers(4) == 0 else int(rs.integers(4))
        slot = MISS if rs.integers(2) == 0 else (MISS - 1 if rs.integers(16) == 0 else int(rs.integers(1 << 20)))
        route[i] = (e, t, slot)
    nw = (experts + 31) // 32
    dens = rs.integers(4)
    words = [np.zeros(nw), np.full(nw, 0xFFFFFFFF), rs.integers(0, 2**32, nw),
             rs.integers(0, 2**32, nw) & rs.integers(0, 2**32, nw)][dens].astype(np.uint32)
    b_copy = [0, 0xFFFFFFFF, int(rs.integers(1 << 20)), int(rs.integers(2**32))][rs.integers(4)]
    eb = [0, int(rs.integers(1, 1 << 16)), int(rs.integers(1, 1 << 24)), int(rs.integers(2**63)) * 2 + 1,
          b_copy][rs.integers(5)]
    slots = [0, int(rs.integers(8)), 0xFFFFFFFF, int(rs.integers(n + 1))][rs.integers(4)]
    return route, (words if nw else np.zeros(1, np.uint32)), experts, b_copy, eb, slots


def test_assign_equals_oracle_on_drawn_inputs(M):
    rs = np.random.default_rng(0x5EED)
    announce("assign drawn inputs")
    copies = 0
    for case in range(600):
        route, words, experts, b_copy, eb, slots = draw_case(rs)
        want = o.moe_assign(route, words if experts else None, experts, b_copy, eb, slots).tolist()
        got = gpu_codes(M, route, words, experts, b_copy, eb, slots)
        assert got == want, f"case {case}: n={len(route)} experts={experts} b={b_copy} eb={eb} slots={slots}"
        copies += sum(c < CPU for c in want)
    assert copies > 300


@pytest.mark.parametrize("n", [1023, 1024, 1025, 5000, 65535])
def test_assign_many_entries(M, n):
    """Several LDS tiles and workgroups: ties, repeats and every class at the largest sizes."""
    rs = np.random.default_rng(n)
    route = np.zeros(n, o.ROUTE_SLOT)
    route["expert"] = rs.integers(0, 3000, n)
    route["tokens"] = rs.integers(0, 5, n)
    route["cache_slot"] = np.where(rs.random(n) < 0.6, MISS, rs.integers(0, 1 << 20, n))
    words = (rs.integers(0, 2**32, 94) & rs.integers(0, 2**32, 94)).astype(np.uint32)
    announce(f"assign n={n}")
    for b_copy, eb, slots in [(0xFFFFFFFF, 1000, 0xFFFFFFFF), (50_000, 100, 300), (0, 0, n // 3)]:
        want = o.moe_assign(route, words, 3000, b_copy, eb, slots).tolist()
        assert gpu_codes(M, route, words, 3000, b_copy, eb, slots) == want


def test_assign_worked_examples(M):
    """crates/kernels/src/moe/tests.rs:801-902 on the device."""
    def run(entries, words, experts, b, eb, slots):
        return gpu_codes(M, o.route_slots(entries), np.array(words or [0], np.uint32), experts, b, eb, slots)

    announce("assign worked examples")
    route = [(7, 3, MISS), (4, 2, 11), (2, 1, MISS), (5, 3, MISS), (9, 1, MISS)]
    words = [1 << 2 | 1 << 5 | 1 << 7]
    assert run(route, words, 16, 200, 100, 8) == [1, HIT, CPU, 0, CPU]
    assert run(route, words, 16, 300, 100, 8) == [1, HIT, 2, 0, CPU]
    assert run(route, words, 16, 300, 100, 1) == [CPU, HIT, CPU, 0, CPU]
    assert run([(9, 2, MISS), (3, 2, MISS), (6, 2, MISS)], [0xFFFFFFFF], 32, 0xFFFFFFFF, 1, 2) == [CPU, 0, 1]
    assert run([(4, 1, MISS)] * 3, [0xFFFFFFFF], 32, 0xFFFFFFFF, 1, 2) == [0, 1, CPU]
    assert run([(0, 1, MISS), (1, 1, 3)], None, 0, 0xFFFFFFFF, 1, 4) == [CPU, HIT]
    got = run([(e, 1, MISS) for e in range(10)], [0xFFFFFFFF], 4, 0xFFFFFFFF, 1, 0xFFFFFFFF)
    assert got == [e if e < 4 else CPU for e in range(10)]
    forty = [(e, 1, MISS) for e in range(40)]
    allw = [0xFFFFFFFF] * 2
    for b, eb, slots, n in [(0xFFFFFFFF, 2**64 - 1, 0xFFFFFFFF, 0), (0xFFFFFFFF, 2**32, 9, 0),
                            (0xFFFFFFFF, 2**32 - 1, 9, 1), (0, 0, 7, 7), (0xFFFFFFFF, 1, 0, 0), (0, 1, 9, 0)]:
        assert sum(c < CPU for c in run(forty, allw, 64, b, eb, slots)) == n


# ---- the doorbell ---------------------------------------------------------------------------
def step_desc(step: int, rows_active: int) -> torch.Tensor:
    d = np.zeros(64, np.uint8)
    d[:8] = np.frombuffer(np.uint64(step).tobytes(), np.uint8)
    d[8:12] = np.frombuffer(np.uint32(rows_active).tobytes(), np.uint8)
    return dev(d)


def check_layer(got, want, max_union, what):
    n = int(want[4:6].view(np.uint16)[0])
    end = 8 + 8 * n
    assert got[:end].tolist() == want[:end].tolist(), what
    assert (got[end:8 + 8 * max_union] == 0xAA).all(), f"{what}: route entries past n_route written"


@pytest.mark.parametrize("rows,top_k,E", [(1, 1, 4), (37, 4, 16), (64, 8, 128), (600, 2, 256),
                                          (3, 8, 8192), (2000, 8, 128), (65535, 1, 300)])
def test_doorbell_equals_oracle(M, rows, top_k, E):
    rs = np.random.default_rng(rows + E)
    ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]) if rows < 5000 else \
        rs.integers(0, E, (rows, top_k))
    ids = ids.astype(np.int32)
    if top_k > 1:
        ids[0, 1] = ids[0, 0]  # a repeat within a row counts the row once
    slot_of = np.where(rs.random(E) < 0.4, MISS, rs.integers(0, 1 << 20, E)).astype(np.uint32)
    max_union = min(E, rows * top_k)
    want = o.moe_doorbell(ids, E, max_union, slot_of, seq=0x12345678)
    layer = torch.full((8 + 8 * max_union + 16,), 0xAA, dtype=torch.uint8, device="cuda")
    st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    announce(f"doorbell rows={rows} k={top_k} E={E}")
    M.doorbell(dev(ids), E, max_union, dev(slot_of), seq=0x12345678, layer=layer, status=st)
    assert int(host(st)[0]) == 0
    got = host(layer)
    check_layer(got, want, max_union, "layer")
    assert (got[8 + 8 * max_union:] == 0xAA).all()


def test_doorbell_reads_the_step_descriptor(M):
    """seq = the low 32 bits of syn_step_desc.step and the rows bounded by its rows_active."""
    rs = np.random.default_rng(12)
    rows, top_k, E = 50, 4, 64
    ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
    announce("doorbell step descriptor")
    for active in (50, 17, 0):
        layer = torch.full((8 + 8 * E,), 0xAA, dtype=torch.uint8, device="cuda")
        M.doorbell(dev(ids), E, E, None, seq=1, step_desc=step_desc((7 << 32) | 0xCAFE0000 | active, active),
                   layer=layer)
        want = o.moe_doorbell(ids[:active], E, E, None, seq=0xCAFE0000 | active)
        check_layer(host(layer), want, E, f"rows_active {active}")


def test_doorbell_refusals_write_nothing(M):
    announce("doorbell refusals")
    for ids, E, max_union, code in [(np.array([[0, 4]], np.int32), 4, 4, 1),
                                     (np.array([[0, 1], [2, 3]], np.int32), 4, 3, 2)]:
        layer = torch.full((8 + 8 * 4,), 0xAA, dtype=torch.uint8, device="cuda")
        st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
        M.doorbell(dev(ids), E, max_union, None, layer=layer, status=st)
        assert int(host(st)[0]) == code
        assert (host(layer) == 0xAA).all()


# ---- codes from the doorbell, and the three sites ------------------------------------------------
def test_assign_layer_reads_n_route_and_b_copy_on_the_device(M):
    rs = np.random.default_rng(21)
    rows, top_k, E = 40, 4, 64
    ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
    slot_of = np.where(rs.random(E) < 0.5, MISS, rs.integers(0, 100, E)).astype(np.uint32)
    words = rs.integers(0, 2**32, 2).astype(np.uint32)
    layer = M.doorbell(dev(ids), E, E, dev(slot_of))
    want_layer = o.moe_doorbell(ids, E, E, slot_of)
    n = int(want_layer[4:6].view(np.uint16)[0])
    route = want_layer[8:8 + 8 * n].view(o.ROUTE_SLOT)
    announce("assign_layer")
    for b in (0, 3000, 0xFFFFFFFF):
        out = torch.full((E,), 0x3A3A3A3A, dtype=torch.int32, device="cuda")
        M.assign_layer(layer, E, dev(words), E, dev(np.array([b], np.uint32)), 1000, 5, out=out)
        got = host(out).view(np.uint32)
        assert got[:n].tolist() == o.moe_assign(route, words, E, b, 1000, 5).tolist()
        assert (got[n:] == 0x3A3A3A3A).all()
    # a header above max_union is refused: no code written
    out = torch.full((E,), 0x3A3A3A3A, dtype=torch.int32, device="cuda")
    M.assign_layer(layer, n - 1, dev(words), E, dev(np.array([0], np.uint32)), 1000, 5, out=out)
    assert (host(out).view(np.uint32) == 0x3A3A3A3A).all()


def test_captured_doorbell_and_codes_follow_the_step(M):
    """One capture of doorbell + codes, replayed with new ids, step number, rows_active and
    B_copy written between replays; every replay equals the oracle."""
    rs = np.random.default_rng(33)
    rows, top_k, E = 24, 4, 32
    ids_d = torch.zeros((rows, top_k), dtype=torch.int32, device="cuda")
    desc = step_desc(0, rows)
    b_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    slot_of = np.where(rs.random(E) < 0.5, MISS, rs.integers(0, 100, E)).astype(np.uint32)
    words = rs.integers(0, 2**32, 1).astype(np.uint32)
    so_d, w_d = dev(slot_of), dev(words)
    layer = torch.zeros(8 + 8 * E, dtype=torch.uint8, device="cuda")
    codes = torch.zeros(E, dtype=torch.int32, device="cuda")
    announce("split capture/replay")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        M.doorbell(ids_d, E, E, so_d, step_desc=desc, layer=layer)
        M.assign_layer(layer, E, w_d, E, b_d, 64, 6, out=codes)
    for rep, (active, b) in enumerate([(24, 200), (9, 0xFFFFFFFF), (0, 100), (24, 0)]):
        ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
        ids_d.copy_(dev(ids))
        desc.copy_(step_desc(1000 + rep, active))
        b_d.copy_(dev(np.array([b], np.uint32).view(np.int32)))
        layer.fill_(0xAA)
        torch.cuda.synchronize()
        g.replay()
        want = o.moe_doorbell(ids[:active], E, E, slot_of, seq=1000 + rep)
        check_layer(host(layer), want, E, f"replay {rep}")
        n = int(want[4:6].view(np.uint16)[0])
        route = want[8:8 + 8 * n].view(o.ROUTE_SLOT)
        got = host(codes).view(np.uint32)[:n].tolist()
        assert got == o.moe_assign(route, words, E, b, 64, 6).tolist(), f"replay {rep}"


@pytest.mark.parametrize("rows,E,top_k,hidden,inter", [(37, 16, 4, 512, 256), (200, 6, 2, 256, 512)])
def test_three_sites_complete_the_layer(M, rows, E, top_k, hidden, inter):
    """route -> doorbell -> codes -> one site mask per class -> MoeGrouped per class on one
    output: every slot is written by exactly its expert's class, and the union equals the
    unmasked layer (RFC-0040 3.4's steps 1-7 on one device)."""
    from test_gpu_moe import fast_q4k_experts
    s = M.MoeShape(E, top_k, hidden, inter)
    gate, up, down = fast_q4k_experts(4, E, hidden, inter)
    ex = M.Experts(12, dev(gate), dev(up), dev(down))
    router = o.normal(0x51A30007, 0.02, E * hidden).reshape(E, hidden)
    x = o.normal(0x51A20007 + rows, 1.0, rows * hidden).reshape(rows, hidden)
    rs = np.random.default_rng(rows)
    slot_of = np.where(rs.random(E) < 0.4, MISS, rs.integers(0, 64, E)).astype(np.uint32)
    words = rs.integers(0, 2**32, (E + 31) // 32).astype(np.uint32)
    eb = 3 * inter * (hidden // 256) * 144
    max_union = min(E, rows * top_k)
    announce(f"three sites rows={rows} E={E}")
    ids_d, w_d = M.route(dev(router), dev(x), top_k, True)
    layer = M.doorbell(ids_d, E, max_union, dev(slot_of), seq=5)
    codes = M.assign_layer(layer, max_union, dev(words), E, dev(np.array([2 * eb], np.uint32)), eb, 4)
    out = torch.full((rows, top_k, hidden), SENTINEL, dtype=torch.int32, device="cuda").view(torch.float32)
    classes = []
    for which in (M.HIT, M.COPY, M.CPU):
        site = M.site_mask(layer, max_union, codes, E, which)
        classes.append(host(site).copy())
        M.moe_grouped(s, ex, dev(x), ids_d, out=out, site=site)
    ids = host(ids_d)
    want_layer = o.moe_doorbell(ids, E, max_union, slot_of, seq=5)
    n = int(want_layer[4:6].view(np.uint16)[0])
    route = want_layer[8:8 + 8 * n].view(o.ROUTE_SLOT)
    want_codes = o.moe_assign(route, words, E, 2 * eb, eb, 4)
    cls = np.zeros((3, E), np.int32)
    for r, c in zip(route, want_codes):
        cls[0 if c == HIT else 2 if c == CPU else 1, r["expert"]] = 1
    assert (np.array(classes) == cls).all()
    assert (cls.sum(0) == (np.bincount(ids.ravel(), minlength=E) > 0)).all()  # each routed expert once
    assert (cls[1].sum() == min(2, int(((slot_of == MISS) & cls.any(0).astype(bool) &
                                       ((words[np.arange(E) // 32] >> (np.arange(E) % 32)) & 1).astype(bool)).sum())))
    want = o.moe_grouped(o.Q4_K, o.Q4_K, E, top_k, hidden, inter, gate, up, down, x, ids, threads=8)
    assert_same(host(out), want, "three sites")
