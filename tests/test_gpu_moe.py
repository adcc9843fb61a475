"""GPU parity of the MoE layer (route, pack, grouped expert FFN, combine) against the CPU oracle:
bit-exact ids, lists and outputs."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from refgen import MoeRng, moe_activations, moe_matrix, moe_route_ids

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    require_gpu()
    import syntropy_amd.moe as M
    return M


def random_q4k_experts(seed, n_experts, hidden, inter):
    """Stacked Q4_K experts as the reference's MoE tests build them (random codes, F16 scales in
    [2^-9, 2^-5]; crates/kernels-cpu/src/moe/tests.rs:40-74)."""
    rng = MoeRng(seed)
    gate = moe_matrix(rng, o.Q4_K, n_experts * inter, hidden, o.f16_bits)
    up = moe_matrix(rng, o.Q4_K, n_experts * inter, hidden, o.f16_bits)
    down = moe_matrix(rng, o.Q4_K, n_experts * hidden, inter, o.f16_bits)
    return gate, up, down


def fast_q4k_experts(seed, n_experts, hidden, inter):
    """The same distribution generated vectorized (for the layer-size cases)."""
    rs = np.random.default_rng(seed)

    def mat(n_out, k):
        nb = n_out * k // 256
        b = np.frombuffer(rs.bytes(nb * 144), np.uint8).reshape(nb, 144).copy()
        # F16 scales in [2^-10, 2^-5): biased exponent 5..9, random mantissa
        h = ((rs.integers(5, 10, (nb, 2), dtype=np.uint16) << 10)
             | rs.integers(0, 1024, (nb, 2), dtype=np.uint16)).astype(np.uint16)
        b[:, 0:4] = h.view(np.uint8).reshape(nb, 4)
        return b.ravel()

    return mat(n_experts * inter, hidden), mat(n_experts * inter, hidden), mat(n_experts * hidden, inter)


# ---- route ----------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,hidden,n_experts,top_k", [
    (37, 256, 16, 4), (64, 4096, 128, 8), (5, 1024, 60, 6), (600, 512, 32, 2),
    # odd block counts at some tree level: 5 and 48 router blocks, 3 softmax blocks
    (9, 160, 70, 5), (300, 1536, 70, 4),
    # the widest rows (fewer experts per workgroup) and 256 experts
    (3, 8192, 40, 3), (5, 7168, 256, 8),
    # 512 rows and more: the many-token kernel (16 x 16 tiles, the tree as a binary stack):
    # the prefill shape, 5 and 224 blocks, experts not a multiple of 16, 256 blocks (9 levels)
    (2048, 4096, 128, 8), (700, 160, 70, 5), (513, 7168, 40, 3), (1000, 8192, 256, 8),
    # one 32-value block (the tree is that block's sum), both kernels; 7 and 31 blocks (partial
    # 8-block chunks of the many-token kernel)
    (10, 32, 8, 2), (600, 32, 20, 3), (520, 224, 33, 4), (530, 992, 17, 1)])
def test_route_bit_exact(M, rows, hidden, n_experts, top_k):
    router = o.normal(0x51A30004 + hidden, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    x = o.normal(0x51A20004 + rows, 1.0, rows * hidden).reshape(rows, hidden)
    announce(f"route rows={rows} hidden={hidden} E={n_experts} k={top_k}")
    ids, w, probs = M.route(dev(router), dev(x), top_k, True, probs=True)
    wids, ww, wprobs = o.moe_route(router, x, n_experts, top_k, True)
    assert_same(host(probs), wprobs, "probs")
    assert (host(ids) == wids).all()
    assert_same(host(w), ww, "weights")


@pytest.mark.parametrize("rows,hidden,n_experts", [(7, 2080, 19), (130, 4096, 128)])
def test_route_token_rows_not_16_byte_aligned(M, rows, hidden, n_experts):
    """Token rows at a 4-byte offset take the 4-byte copy path; a hidden size of 65 blocks
    leaves a one-block last chunk."""
    router = o.normal(0x51A30004 + hidden, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    x = o.normal(0x51A20004 + rows, 1.0, rows * hidden).reshape(rows, hidden)
    flat = torch.empty(rows * hidden + 1, dtype=torch.float32, device="cuda")
    xs = flat[1:].view(rows, hidden)
    xs.copy_(torch.from_numpy(x))
    assert xs.data_ptr() % 16 == 4
    announce(f"route misaligned rows={rows} hidden={hidden} E={n_experts}")
    ids, w, probs = M.route(dev(router), xs, 4, True, probs=True)
    wids, ww, wprobs = o.moe_route(router, x, n_experts, 4, True)
    assert_same(host(probs), wprobs, "probs")
    assert (host(ids) == wids).all()
    assert_same(host(w), ww, "weights")


def test_route_nan_rows_match_the_first_best_scan(M):
    """A NaN logit makes every probability of its row NaN (the F32Fixed sum is NaN); the
    selection is then experts 0..k-1, as the oracle's first-best scan gives, and the weights
    are NaN.  Rows without NaN are unaffected."""
    hidden, n_experts, rows = 256, 40, 9
    router = o.normal(21, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    x = o.normal(22, 1.0, rows * hidden).reshape(rows, hidden)
    x[2, 7] = np.nan
    router[0, 3] = np.nan  # logit 0 NaN in every row: the row maximum itself is NaN
    x2 = x.copy()
    announce("route nan")
    for r in (router, router * np.float32(1)):
        ids, w, probs = M.route(dev(r), dev(x2), 5, True, probs=True)
        wids, ww, wprobs = o.moe_route(r, x2, n_experts, 5, True)
        assert (host(ids) == wids).all()
        assert_same(host(w), ww, "weights")
        assert_same(host(probs), wprobs, "probs")
    r = router.copy()
    r[0, 3] = 0.5
    ids, w, probs = M.route(dev(r), dev(x), 5, True, probs=True)
    wids, ww, wprobs = o.moe_route(r, x, n_experts, 5, True)
    assert (host(ids) == wids).all() and (wids[2] == np.arange(5)).all()
    assert_same(host(w), ww, "weights")
    assert np.isnan(host(w)[2]).all() and not np.isnan(host(w)[[0, 1, 3]]).any()


def test_route_ties_go_to_the_lower_index(M):
    hidden, n_experts = 256, 16
    router = o.normal(3, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    router[9] = router[2]
    router[11] = router[2]
    router[5] = router[14]
    x = o.normal(4, 1.0, 8 * hidden).reshape(8, hidden)
    announce("route ties")
    ids, w = M.route(dev(router), dev(x), 6, True)
    wids, ww, _ = o.moe_route(router, x, n_experts, 6, True)
    assert (host(ids) == wids).all()
    assert_same(host(w), ww)
    # brute force: the selection is the stable descending sort of the probabilities
    _, _, p = o.moe_route(router, x, n_experts, 6, True)
    for r in range(8):
        order = sorted(range(n_experts), key=lambda e: (-p[r, e], e))[:6]
        assert list(host(ids)[r]) == order


# ---- pack -------------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,top_k,n_experts", [(1, 1, 4), (64, 8, 128), (2048, 8, 128),
                                                   (300, 3, 7), (17, 2, 256)])
def test_pack_bit_exact(M, rows, top_k, n_experts):
    rs = np.random.default_rng(rows * 31 + top_k)
    ids = rs.integers(0, n_experts, (rows, top_k)).astype(np.int32)
    if rows >= 64:  # skew: a few experts take many slots
        ids[: rows // 2, 0] = 3
    announce(f"pack rows={rows} k={top_k} E={n_experts}")
    offsets, slots, err = M.pack(dev(ids), n_experts)
    wo, ws = o.moe_pack(ids, n_experts)
    assert host(err)[0] == 0
    assert (host(offsets).view(np.uint32) == wo).all()
    assert (host(slots).view(np.uint32) == ws).all()


def test_pack_refuses_bad_ids(M):
    ids = np.zeros((8, 2), np.int32)
    ids[5, 1] = 9
    announce("pack bad id")
    _, _, err = M.pack(dev(ids), 9)
    assert host(err)[0] == 1


# ---- grouped expert FFN ------------------------------------------------------------------------
LAYOUTS = (0, 3)  # the experts in GGUF order and in TILE64


def tile64_numpy(w, k):
    """TILE64 by its definition: each run of 64 rows of k / 256 super-blocks, block-major."""
    return w.reshape(-1, 64, k // 256, 144).transpose(0, 2, 1, 3).ravel()


def run_grouped(M, shape, gate, up, down, x, ids, layout=0):
    ex = M.Experts(12, dev(gate), dev(up), dev(down))
    if layout:
        ex = M.tile64(ex, shape)
        assert ex.layout == layout
    out = torch.full((ids.shape[0], shape.top_k, shape.hidden), float("nan"), device="cuda")
    st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    M.moe_grouped(shape, ex, dev(x), dev(ids), out=out, status=st)
    return host(out), int(host(st)[0])


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("rows", [1, 2, 5, 8, 9, 17, 40])
def test_grouped_equals_oracle_reference_shape(M, rows, layout):
    """crates/kernels-cpu/src/moe/tests.rs:227-236 shape: 6 experts, top-2, hidden 256, inter 512;
    the experts in GGUF order and in TILE64."""
    s = M.MoeShape(6, 2, 256, 512)
    gate, up, down = random_q4k_experts(1, s.n_experts, s.hidden, s.inter)
    rng = MoeRng(100 + rows)
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    announce(f"grouped ref-shape rows={rows} layout={layout}")
    got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 6, 2, 256, 512, gate, up, down, x, ids)
    assert st == 0
    assert_same(got, want, f"rows {rows}")


def test_grouped_layer_shape_64_tokens(M):
    """Qwen3-235B-A22B MoE shape at 64 decode tokens: 128 experts, top-8, hidden 4096, inter 1536,
    routed by the GPU router on N(0,1) rows; every slot bit-exact against the oracle."""
    s = M.MoeShape(128, 8, 4096, 1536)
    gate, up, down = fast_q4k_experts(7, s.n_experts, s.hidden, s.inter)
    router = o.normal(0x51A30004, 0.02, s.n_experts * s.hidden).reshape(s.n_experts, s.hidden)
    x = o.normal(0x51A20004, 1.0, 64 * s.hidden).reshape(64, s.hidden)
    announce("grouped layer shape 64 tokens")
    ids_d, w_d = M.route(dev(router), dev(x), s.top_k, True)
    ids = host(ids_d)
    wids, ww, _ = o.moe_route(router, x, s.n_experts, s.top_k, True)
    assert (ids == wids).all()
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 128, 8, 4096, 1536, gate, up, down, x, ids, threads=16)
    for layout in LAYOUTS:
        announce(f"grouped layer shape 64 tokens layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 0
        assert_same(got, want, f"layer slots, layout {layout}")
    y = host(M.combine(dev(got), dev(ids), dev(ww)))
    assert_same(y, o.moe_combine(want, ids, ww), "combined")


def test_moe_layer_2048_skewed_tokens(M):
    """The prefill MoE layer: 2048 tokens, 128 experts, top-8, hidden 4096, inter 1536, with
    router rows 3, 50 and 97 scaled by 3 so those experts take over four times the average load.
    Route, the grouped FFN (the many-token path) and the combine, every value against the oracle."""
    s = M.MoeShape(128, 8, 4096, 1536)
    T = 2048
    gate, up, down = fast_q4k_experts(0x51A4, s.n_experts, s.hidden, s.inter)
    router = o.normal(0x51A30004, 0.02, s.n_experts * s.hidden).reshape(s.n_experts, s.hidden)
    for r in (3, 50, 97):
        router[r] *= np.float32(3.0)
    x = o.normal(0x51A20005, 1.0, T * s.hidden).reshape(T, s.hidden)
    announce("moe layer 2048 skewed tokens: route")
    ids_d, w_d = M.route(dev(router), dev(x), s.top_k, True)
    wids, ww, _ = o.moe_route(router, x, s.n_experts, s.top_k, True)
    ids = host(ids_d)
    assert (ids == wids).all()
    assert_same(host(w_d), ww, "weights")
    loads = np.sort(np.bincount(ids.ravel(), minlength=s.n_experts))[::-1]
    assert (loads[:3] >= 4 * T * s.top_k / s.n_experts).all(), loads[:4]
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 128, 8, 4096, 1536, gate, up, down, x, ids, threads=16)
    for layout in LAYOUTS:
        announce(f"moe layer 2048 skewed tokens: grouped, layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 0
        assert_same(got, want, f"slots, layout {layout}")
    announce("moe layer 2048 skewed tokens: combine")
    y = host(M.combine(dev(got), dev(ids), dev(ww)))
    assert_same(y, o.moe_combine(want, ids, ww), "combined")


def test_grouped_skewed_loads(M):
    """One expert takes most rows (more entries than one work item holds)."""
    s = M.MoeShape(8, 2, 512, 256)
    gate, up, down = random_q4k_experts(5, s.n_experts, s.hidden, s.inter)
    rows = 150
    rng = MoeRng(9)
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    ids[:120, 0] = 6
    ids[:120, 1] = np.where(ids[:120, 1] == 6, 2, ids[:120, 1])
    announce("grouped skewed")
    got, st = run_grouped(M, s, gate, up, down, x, ids)
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 8, 2, 512, 256, gate, up, down, x, ids)
    assert st == 0
    assert_same(got, want)


def test_grouped_decode_path_heavy_expert(M):
    """The decode kernels (few entries per expert on average) with one expert holding 35 of 80
    entries: its entries span several work items of the gate/up (16 entries) and down (12
    entries) kernels, the last one partial and starting off a multiple of four."""
    s = M.MoeShape(16, 2, 512, 768)
    gate, up, down = random_q4k_experts(21, s.n_experts, s.hidden, s.inter)
    rows = 40
    rng = MoeRng(23)
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    ids[:35, 0] = 3
    ids[:35, 1] = np.where(ids[:35, 1] == 3, 11, ids[:35, 1])
    ids[35] = [0, 2]
    counts = np.bincount(ids.ravel(), minlength=s.n_experts)
    assert counts[3] == 35 and counts[:3].sum() % 4 == 2  # expert 3's entries start at 6
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 16, 2, 512, 768, gate, up, down, x, ids)
    for layout in LAYOUTS:
        announce(f"grouped decode path heavy expert layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 0
        assert_same(got, want, f"layout {layout}")


def test_grouped_row_permutation(M):
    """moe/tests.rs:497-539: permuting rows permutes the per-slot and combined outputs."""
    s = M.MoeShape(6, 2, 256, 512)
    gate, up, down = random_q4k_experts(2, s.n_experts, s.hidden, s.inter)
    rng = MoeRng(5)
    rows = 12
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    w = np.array([abs(rng.unit()) for _ in range(rows * s.top_k)], np.float32).reshape(rows, s.top_k)
    perm = [(rows - 1 - i) for i in range(rows)]
    perm = perm[rows // 3:] + perm[:rows // 3]
    announce("grouped permutation")
    out, _ = run_grouped(M, s, gate, up, down, x, ids)
    outp, _ = run_grouped(M, s, gate, up, down, x[perm], ids[perm])
    assert_same(outp, out[perm])
    y = host(M.combine(dev(out), dev(ids), dev(w)))
    yp = host(M.combine(dev(outp), dev(ids[perm]), dev(w[perm])))
    assert_same(yp, y[perm])


# ---- the grouped FFN on the prefill GEMM (experts averaging 32 or more entries) ---------------
@pytest.mark.parametrize("rows", [96, 200, 333])
def test_grouped_gemm_path_equals_oracle(M, rows):
    """The reference test shape at token counts that take the matrix-core GEMM path: entries
    padded to 64-entry tiles per expert, gate and up in one workgroup, down to the slots."""
    s = M.MoeShape(6, 2, 256, 512)
    gate, up, down = random_q4k_experts(2, s.n_experts, s.hidden, s.inter)
    rng = MoeRng(300 + rows)
    x = moe_activations(rng, rows * s.hidden).reshape(rows, s.hidden)
    ids = moe_route_ids(rng, rows, s.top_k, s.n_experts)
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 6, 2, 256, 512, gate, up, down, x, ids)
    for layout in LAYOUTS:
        announce(f"grouped gemm path rows={rows} layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 0
        assert_same(got, want, f"rows {rows}, layout {layout}")


def test_grouped_gemm_path_skewed_and_empty_experts(M):
    """One expert takes 300 entries (five tiles, the last partial), four take none, and the
    hidden size spans several 256-row down tiles and 128-row gate/up tiles."""
    s = M.MoeShape(16, 4, 1024, 512)
    gate, up, down = fast_q4k_experts(5, s.n_experts, s.hidden, s.inter)
    rows = 160
    rs = np.random.default_rng(9)
    x = rs.standard_normal((rows, s.hidden)).astype(np.float32)
    ids = np.stack([rs.permutation(12)[: s.top_k] for _ in range(rows)]).astype(np.int32)  # experts 12-15 empty
    ids[:, 0] = np.where(np.arange(rows) < 150, 3, ids[:, 0])
    for r in range(rows):  # distinct experts per row
        for j in range(1, s.top_k):
            if ids[r, j] in ids[r, :j]:
                ids[r, j] = next(e for e in range(12) if e not in ids[r])
    cnt = np.bincount(ids.ravel(), minlength=16)
    assert cnt[3] >= 150 and (cnt[12:] == 0).all()
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 16, 4, 1024, 512, gate, up, down, x, ids, threads=8)
    for layout in LAYOUTS:
        announce(f"grouped gemm path skewed layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 0
        assert_same(got, want, f"skewed, layout {layout}")


def test_grouped_gemm_path_refusal_writes_nothing(M):
    s = M.MoeShape(4, 2, 256, 256)
    gate, up, down = random_q4k_experts(3, s.n_experts, s.hidden, s.inter)
    rows = 80
    x = np.ones((rows, 256), np.float32)
    ids = np.tile(np.array([[0, 1]], np.int32), (rows, 1))
    ids[41, 1] = 4
    for layout in LAYOUTS:
        announce(f"grouped gemm path bad id layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 1
        assert np.isnan(got).all()


def test_grouped_refusal_writes_nothing(M):
    s = M.MoeShape(6, 2, 256, 512)
    gate, up, down = random_q4k_experts(3, s.n_experts, s.hidden, s.inter)
    x = np.ones((3, 256), np.float32)
    ids = np.array([[0, 1], [2, 6], [3, 4]], np.int32)
    for layout in LAYOUTS:
        announce(f"grouped bad id layout={layout}")
        got, st = run_grouped(M, s, gate, up, down, x, ids, layout)
        assert st == 1
        assert np.isnan(got).all()


@pytest.mark.parametrize("rows,n_experts,top_k", [(3, 256, 1), (40, 256, 8), (300, 4, 1)])
def test_grouped_extreme_expert_counts(M, rows, n_experts, top_k):
    """256 experts (the largest) with top-1 and top-8 at decode sizes, and top-1 over 4 experts
    on the many-token path (75 entries per expert)."""
    s = M.MoeShape(n_experts, top_k, 256, 256)
    gate, up, down = fast_q4k_experts(13 + rows, n_experts, 256, 256)
    rs = np.random.default_rng(rows + n_experts)
    x = rs.standard_normal((rows, 256)).astype(np.float32)
    ids = np.stack([rs.permutation(n_experts)[:top_k] for _ in range(rows)]).astype(np.int32)
    announce(f"grouped E={n_experts} k={top_k} rows={rows}")
    got, st = run_grouped(M, s, gate, up, down, x, ids)
    assert st == 0
    want = o.moe_grouped(o.Q4_K, o.Q4_K, n_experts, top_k, 256, 256, gate, up, down, x, ids, threads=8)
    assert_same(got, want, "extreme experts")


# ---- the site mask (MoeGrouped's input 2) ------------------------------------------------------
SENTINEL = 0x7FC0DEAD


@pytest.mark.parametrize("rows,n_experts,top_k,hidden,inter", [
    (6, 6, 2, 256, 512),       # moe/tests.rs:559-590, on the decode kernels
    (64, 128, 8, 4096, 1536),  # the 64-token layer shape, decode kernels
    (200, 6, 2, 256, 512),     # the many-token GEMM path
    (160, 16, 4, 1024, 512)])  # GEMM path, several row tiles
def test_grouped_site_mask(M, rows, n_experts, top_k, hidden, inter):
    """Experts the site mask leaves out are not computed: their slots keep their bits, the rest
    equal the oracle's; the complementary call on the same output completes the unmasked one."""
    s = M.MoeShape(n_experts, top_k, hidden, inter)
    gate, up, down = fast_q4k_experts(11, n_experts, hidden, inter)
    rs = np.random.default_rng(rows)
    x = rs.standard_normal((rows, hidden)).astype(np.float32)
    ids = np.stack([rs.permutation(n_experts)[:top_k] for _ in range(rows)]).astype(np.int32)
    site = (rs.random(n_experts) < 0.5).astype(np.int32)
    site[ids[0, 0]] = 1
    site[ids[0, 1]] = 0
    args = (o.Q4_K, o.Q4_K, n_experts, top_k, hidden, inter, gate, up, down, x, ids)
    want = o.moe_grouped(*args, site=site, threads=8,
                         out=np.full(rows * top_k * hidden, SENTINEL, np.uint32).view(np.float32))
    want_all = o.moe_grouped(*args, threads=8)
    kept = site[ids] == 0
    ex0 = M.Experts(12, dev(gate), dev(up), dev(down))
    for ex in (ex0, M.tile64(ex0, s)):
        out = torch.full((rows, top_k, hidden), SENTINEL, dtype=torch.int32, device="cuda").view(torch.float32)
        st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
        announce(f"grouped site rows={rows} E={n_experts} k={top_k} hidden={hidden} inter={inter} "
                 f"layout={ex.layout}")
        M.moe_grouped(s, ex, dev(x), dev(ids), out=out, status=st, site=dev(site))
        got = host(out)
        assert int(host(st)[0]) == 0
        assert_same(got, want, f"masked, layout {ex.layout}")
        assert (got[kept].view(np.uint32) == SENTINEL).all()
        M.moe_grouped(s, ex, dev(x), dev(ids), out=out, status=st, site=dev(1 - site))
        assert_same(host(out), want_all, f"both sites, layout {ex.layout}")


# ---- the TILE64 expert layout ---------------------------------------------------------------------
@pytest.mark.parametrize("rows,k", [(64, 256), (128, 768), (3 * 1536, 4096)])
def test_tile64_repack_matches_definition_and_inverts(M, rows, k):
    """The device repack places each run's block b of row r at 144 (64 b + r), as the host repack
    does, and its inverse restores the GGUF rows (one stack of 3 experts' gate rows last)."""
    rs = np.random.default_rng(rows + k)
    w = np.frombuffer(rs.bytes(rows * k // 256 * 144), np.uint8).copy()
    announce(f"tile64 repack rows={rows} k={k}")
    t = M.tile64_repack(dev(w), k)
    want = tile64_numpy(w, k)
    assert (host(t) == want).all()
    from syntropy_amd._lib import lib
    viahost = np.empty_like(w)
    assert lib().syn_q4k_tile64_repack_host(w.ctypes.data, viahost.ctypes.data, w.size, k, 0) == 0
    assert (viahost == want).all()
    assert (host(M.tile64_repack(t, k, inverse=True)) == w).all()


def test_tile64_refusals(M):
    """Rows that are not whole 64-row runs, and TILE64 for Q8_0 experts, are refused before any
    launch."""
    w = torch.zeros(100 * 144, dtype=torch.uint8, device="cuda")
    with pytest.raises(Exception, match="whole runs of 64 rows"):
        M.tile64_repack(w, 256)
    s = M.MoeShape(4, 2, 256, 256)
    q8 = torch.zeros(4 * 256 * 8 * 34, dtype=torch.uint8, device="cuda")
    with pytest.raises(M.MoeError, match="layout 3"):
        M.moe_grouped(s, M.Experts(8, q8, q8, q8, M.LAYOUT_TILE64), torch.zeros(1, 256, device="cuda"),
                      torch.zeros(1, 2, dtype=torch.int32, device="cuda"))


# ---- combine ------------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,k,hidden", [(33, 8, 1000), (5, 8, 1001), (64, 8, 4096), (3, 64, 130),
                                          (7, 1, 4096), (2, 3, 2050)])
def test_combine_bit_exact(M, rows, k, hidden):
    """Float4 columns (hidden a multiple of 4) and the scalar tail; top_k 1 to 64; repeated ids
    in a row keep their slot order (the stable sort of moe/tests.rs:541-556)."""
    rs = np.random.default_rng(rows * 31 + hidden)
    out = rs.standard_normal((rows, k, hidden)).astype(np.float32)
    ids = np.stack([rs.permutation(max(64, k))[:k] for _ in range(rows)]).astype(np.int32)
    if k > 2:
        ids[0, 1] = ids[0, 0]
        ids[-1, k - 1] = ids[-1, 0]
    w = rs.random((rows, k)).astype(np.float32)
    announce(f"combine rows={rows} k={k} hidden={hidden}")
    assert_same(host(M.combine(dev(out), dev(ids), dev(w))), o.moe_combine(out, ids, w))
    # an output view 4 bytes into its buffer takes the scalar path
    flat = torch.zeros(rows * k * hidden + 1, device="cuda")
    flat[1:] = dev(out).reshape(-1)
    view = flat[1:].view(rows, k, hidden)
    assert_same(host(M.combine(view, dev(ids), dev(w))), o.moe_combine(out, ids, w), "unaligned")


@pytest.mark.parametrize("rows,k,hidden,n_shared", [(33, 8, 1000, 0), (5, 8, 1001, 1), (64, 8, 4096, 0),
                                                    (3, 64, 130, 3), (7, 1, 4096, 8), (2, 3, 2050, 2)])
def test_combine_ranked_bit_exact(M, rows, k, hidden, n_shared):
    """MoeCombine as the graph binds it: slots in rank order, then the shared outputs; float4
    columns and the scalar tail, top_k 1 to 64, 0 to 8 shared outputs."""
    rs = np.random.default_rng(rows * 37 + hidden + n_shared)
    out = rs.standard_normal((rows, k, hidden)).astype(np.float32)
    w = rs.random((rows, k)).astype(np.float32)
    shared = [rs.standard_normal((rows, hidden)).astype(np.float32) for _ in range(n_shared)]
    announce(f"combine ranked rows={rows} k={k} hidden={hidden} shared={n_shared}")
    want = o.moe_combine_ranked(out, w, shared)
    got = M.combine_ranked(dev(out), dev(w), [dev(a) for a in shared])
    assert_same(host(got), want)
    # views 4 bytes into their buffers take the scalar path
    flat = torch.zeros(rows * k * hidden + 1, device="cuda")
    flat[1:] = dev(out).reshape(-1)
    view = flat[1:].view(rows, k, hidden)
    assert_same(host(M.combine_ranked(view, dev(w), [dev(a) for a in shared])), want, "unaligned")


def test_combine_ranked_refusals(M):
    out, w = torch.zeros(2, 3, 8, device="cuda"), torch.zeros(2, 3, device="cuda")
    with pytest.raises(M.MoeError):
        M.combine_ranked(out, w, [torch.zeros(2, 8, device="cuda")] * 9)
    with pytest.raises(M.MoeError):
        M.combine_ranked(out, w, [torch.zeros(2, 9, device="cuda")])
