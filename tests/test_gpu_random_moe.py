"""The MoE layer over seeded random shapes: expert count, top-k, hidden and intermediate sizes, token
count and expert layout drawn from a fixed seed per case; the router's ids, every slot of the
grouped expert FFN and the rank-order combine bit-identical to the oracle.

The grouped FFN takes the decode expert kernels or, once the entries average 32 an expert, the
many-token GEMM; the token counts are drawn on both sides of that switch, with loads from one
entry an expert to hundreds."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_moe import fast_q4k_experts

pytestmark = pytest.mark.gpu

MAX_EXPERT_WEIGHTS = 320 << 20  # weights of the three stacked matrices, at most
MAX_MACS = 3 << 30              # the oracle's multiply-adds a case, at most


def draw(case: int):
    """(n_experts, top_k, hidden, inter, rows, layout) of one case."""
    rs = np.random.default_rng(0x3E0E00 + case)
    many = case % 2 == 1  # enough entries for the many-token GEMM (32 an expert on average)
    n_experts = int(rs.integers(2, 25 if many else 161))
    top_k = int(rs.integers(1, min(8, n_experts) + 1))
    hidden = 256 * int(rs.integers(1, 9 if many else 17))
    inter = 256 * int(rs.integers(1, 5 if many else 9))
    while n_experts * 3 * hidden * inter > MAX_EXPERT_WEIGHTS:
        n_experts = max(top_k, n_experts // 2)
        if n_experts == top_k:
            hidden = max(256, hidden // 2)
    if many:
        rows = -(-32 * n_experts // top_k) + int(rs.integers(0, 64))
        while rows * top_k * 3 * hidden * inter > MAX_MACS and hidden > 256:
            hidden //= 2
    else:
        rows = int(rs.integers(1, 100))
        rows = max(1, min(rows, MAX_MACS // (top_k * 3 * hidden * inter)))
    layout = 3 if case % 3 == 0 else 0  # TILE64 or GGUF order
    return n_experts, top_k, hidden, inter, rows, layout


@pytest.fixture(scope="module")
def M():
    require_gpu()
    import syntropy_amd.moe as M
    return M


@pytest.mark.parametrize("case", range(40))
def test_random_moe_layer_equals_oracle(M, case):
    n_experts, top_k, hidden, inter, rows, layout = draw(case)
    s = M.MoeShape(n_experts, top_k, hidden, inter)
    gate, up, down = fast_q4k_experts(0x3E0F00 + case, n_experts, hidden, inter)
    router = o.normal(0x3E1000 + case, 0.02, n_experts * hidden).reshape(n_experts, hidden)
    x = o.normal(0x3E1100 + case, 1.0, rows * hidden).reshape(rows, hidden)
    announce(f"random moe case {case}: E={n_experts} k={top_k} hidden={hidden} inter={inter} rows={rows} "
             f"layout={layout}")
    ids_d, w_d = M.route(dev(router), dev(x), top_k, True)
    wids, ww, _ = o.moe_route(router, x, n_experts, top_k, True)
    ids = host(ids_d)
    assert (ids == wids).all(), "route ids"
    assert_same(host(w_d), ww, "route weights")
    ex = M.Experts(12, dev(gate), dev(up), dev(down))
    if layout:
        ex = M.tile64(ex, s)
    out = torch.full((rows, top_k, hidden), float("nan"), device="cuda")
    st = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    M.moe_grouped(s, ex, dev(x), ids_d, out=out, status=st)
    want = o.moe_grouped(o.Q4_K, o.Q4_K, n_experts, top_k, hidden, inter, gate, up, down, x, ids, threads=16)
    assert int(host(st)[0]) == 0
    assert_same(host(out), want, "grouped slots")
    y = host(M.combine_ranked(out, w_d))
    assert_same(y, o.moe_combine_ranked(want, ww), "rank-order combine")
