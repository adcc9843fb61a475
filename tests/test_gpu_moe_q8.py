"""GPU parity of MoeGrouped over Q8_0 experts (crates/kernels-cpu/src/moe/entry.rs:50-55:
Q8_0 gate, up and down with Q8_0 activations) against the oracle, bit for bit: the reference
test shape, the 64-token layer shape, skewed many-token loads, row widths that are not whole
16-block stages, the site mask, a refused id, and the provider's key."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from refgen import MoeRng, moe_activations, moe_matrix, moe_route_ids
from test_gpu_provider import Ctx, shape

pytestmark = pytest.mark.gpu
Q8 = o.Q8_0


@pytest.fixture(scope="module")
def M():
    require_gpu()
    import syntropy_amd.moe as M
    return M


def q8_experts(seed, n_experts, hidden, inter):
    """Stacked Q8_0 experts: random codes, F16 scales with biased exponents 5..9."""
    rs = np.random.default_rng(seed)

    def mat(n_out, k):
        nb = n_out * k // 32
        b = np.frombuffer(rs.bytes(nb * 34), np.uint8).reshape(nb, 34).copy()
        h = ((rs.integers(5, 10, nb, dtype=np.uint16) << 10) | rs.integers(0, 1024, nb, dtype=np.uint16))
        b[:, 0:2] = h.astype(np.uint16).view(np.uint8).reshape(nb, 2)
        return b.ravel()

    return mat(n_experts * inter, hidden), mat(n_experts * inter, hidden), mat(n_experts * hidden, inter)


def run(M, s, gate, up, down, x, ids, site=None, out=None):
    ex = M.Experts(M.WeightType.Q8_0, dev(gate), dev(up), dev(down))
    if out is None:
        out = torch.full((ids.shape[0], s.top_k, s.hidden), float("nan"), device="cuda")
    st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    M.moe_grouped(s, ex, dev(x), dev(ids), out=out, status=st, site=None if site is None else dev(site))
    return host(out), int(host(st)[0])


@pytest.mark.parametrize("rows", [1, 2, 5, 8, 9, 17, 40])
def test_q8_reference_shape(M, rows):
    """crates/kernels-cpu/src/moe/tests.rs:227-236's shape with Q8_0 experts built by the test
    generator (moe/tests.rs:40-74)."""
    s = M.MoeShape(6, 2, 256, 512)
    rng = MoeRng(200 + rows)
    gate = moe_matrix(rng, Q8, s.n_experts * s.inter, s.hidden, o.f16_bits)
    up = moe_matrix(rng, Q8, s.n_experts * s.inter, s.hidden, o.f16_bits)
    down = moe_matrix(rng, Q8, s.n_experts * s.hidden, s.inter, o.f16_bits)
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    announce(f"q8 moe reference shape rows={rows}")
    got, st = run(M, s, gate, up, down, x, ids)
    assert st == 0
    assert_same(got, o.moe_grouped(Q8, Q8, 6, 2, 256, 512, gate, up, down, x, ids), f"rows {rows}")


@pytest.mark.parametrize("rows,n_experts,top_k,hidden,inter", [
    (64, 128, 8, 4096, 1536),  # the 64-token decode layer shape
    (300, 16, 4, 1024, 512),   # many entries per expert, one expert over-loaded
    (33, 8, 3, 160, 352),      # 5 and 11 blocks: partial stages, rows not 16-byte multiples
    (3, 256, 8, 2048, 96),     # 256 experts, mostly empty
])
def test_q8_layer_shapes(M, rows, n_experts, top_k, hidden, inter):
    s = M.MoeShape(n_experts, top_k, hidden, inter)
    gate, up, down = q8_experts(rows + hidden, n_experts, hidden, inter)
    rs = np.random.default_rng(rows)
    x = rs.standard_normal((rows, hidden)).astype(np.float32)
    ids = np.stack([rs.permutation(n_experts)[:top_k] for _ in range(rows)]).astype(np.int32)
    if rows >= 300:
        ids[:250, 0] = 5
        for r in range(rows):
            for j in range(1, top_k):
                if ids[r, j] in ids[r, :j]:
                    ids[r, j] = next(e for e in range(n_experts) if e not in ids[r])
    announce(f"q8 moe rows={rows} E={n_experts} k={top_k} hidden={hidden} inter={inter}")
    got, st = run(M, s, gate, up, down, x, ids)
    assert st == 0
    want = o.moe_grouped(Q8, Q8, n_experts, top_k, hidden, inter, gate, up, down, x, ids, threads=16)
    assert_same(got, want, "q8 layer")


def test_q8_site_mask_and_refusal(M):
    """Masked experts keep their slots' bits and the complementary call completes the output; a
    bad id writes nothing and reports status 1."""
    SENT = 0x7FC0DEAD
    rows, E, top_k, hidden, inter = 40, 12, 3, 512, 256
    s = M.MoeShape(E, top_k, hidden, inter)
    gate, up, down = q8_experts(9, E, hidden, inter)
    rs = np.random.default_rng(4)
    x = rs.standard_normal((rows, hidden)).astype(np.float32)
    ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
    site = (np.arange(E) % 3 != 0).astype(np.int32)
    out = torch.full((rows, top_k, hidden), SENT, dtype=torch.int32, device="cuda").view(torch.float32)
    announce("q8 moe site mask")
    got, st = run(M, s, gate, up, down, x, ids, site=site, out=out)
    assert st == 0
    args = (Q8, Q8, E, top_k, hidden, inter, gate, up, down, x, ids)
    want = o.moe_grouped(*args, site=site, threads=8,
                         out=np.full(rows * top_k * hidden, SENT, np.uint32).view(np.float32))
    assert_same(got, want, "masked")
    assert (got[site[ids] == 0].view(np.uint32) == SENT).all()
    done, _ = run(M, s, gate, up, down, x, ids, site=1 - site, out=out)
    assert_same(done, o.moe_grouped(*args, threads=8), "both sites")
    bad = ids.copy()
    bad[7, 2] = E
    announce("q8 moe bad id")
    got, st = run(M, s, gate, up, down, x, bad)
    assert st == 1 and np.isnan(got).all()


def test_q8_moe_through_the_provider():
    """The provider answers MoeGrouped with Q8_0 experts (Q8Block32 activations, I32ThenF32 over
    32-value blocks, as moe/entry.rs:101-114 declares) and computes the oracle's bits."""
    c = Ctx()
    try:
        P, pr = c.P, c.pr
        E, top_k, hidden, inter, rows = 16, 4, 512, 256, 21
        gate, up, down = q8_experts(77, E, hidden, inter)
        rs = np.random.default_rng(5)
        x = rs.standard_normal((rows, hidden)).astype(np.float32)
        ids = np.stack([rs.permutation(E)[:top_k] for _ in range(rows)]).astype(np.int32)
        key = {"op": "MoeGrouped", "schemes": [{"Ggml": "Q8_0"}, {"Plain": "F32"}, {"Plain": "F32"}],
               "layout": 0, "variant": 0}
        caps = pr.query(c.ctx, key, shape(rows, E, top_k, hidden, inter))
        assert caps["numerics"]["max_block"] == 32 and caps["numerics"]["act_in"] == 2
        assert caps["numerics"]["accumulate"] == 1
        op = pr.prepare(c.ctx, key, shape(rows, E, top_k, hidden, inter))
        gd, ud, dd = dev(gate), dev(up), dev(down)
        views = [P.view(t.data_ptr(), t.numel()) for t in (gd, ud, dd)]
        xb, ib = c.put(x), c.put(ids)
        per_b = c.empty(4 * rows * top_k * hidden)
        announce("provider q8 moe")
        pr.launch(c.ctx, c.s, op, P.op_args([P.packed(xb, P.DT_F32, [rows, hidden]),
                                             P.packed(ib, P.DT_I32, [rows, top_k])],
                                            [P.packed(per_b, P.DT_F32, [rows, top_k, hidden])], views,
                                            c.workspace(op)))
        want = o.moe_grouped(Q8, Q8, E, top_k, hidden, inter, gate, up, down, x, ids, threads=8)
        assert_same(c.get(per_b, np.float32, (rows, top_k, hidden)), want, "provider q8")
    finally:
        c.close()
