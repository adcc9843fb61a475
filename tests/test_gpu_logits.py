"""GPU parity of RmsNorm and Logits (crates/kernels/src/reference/norm.rs:39-47,
crates/kernels/src/reference/linear.rs:118-161) against the oracle, bit for bit: the norm's
F32Fixed sum of squares and its operation order, then the head as the Gemv op, at a vocabulary-
sized head (128256 x 4096) in both Q4_K layouts and Q8_0, directly and through the provider."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_gemm import random_q4k
from test_gpu_provider import Ctx, shape

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 128256, 4096


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


@pytest.mark.parametrize("rows,n", [(1, 4096), (7, 8192), (3, 100), (2, 16384), (5, 32), (4, 33), (9, 7168),
                                    (1, 1)])
def test_rms_norm_bit_exact(S, rows, n):
    """Block counts with an odd carry at several tree levels (100 -> 4 blocks, 7168 -> 224,
    33 -> 2 with a one-value block), one block, and the widest row."""
    rs = np.random.default_rng(rows * 100 + n)
    x = (rs.standard_normal((rows, n)) * 10.0 ** rs.integers(-3, 3, (rows, 1))).astype(np.float32)
    g = (1 + 0.1 * rs.standard_normal(n)).astype(np.float32)
    announce(f"rms_norm rows={rows} n={n}")
    got = host(S.rms_norm(dev(x), dev(g), 1e-5, rows))
    assert_same(got, o.rms_norm(x, g, 1e-5), "rms_norm")


def test_rms_norm_edge_rows(S):
    """norm.rs's documented cases on the device: zeros with eps > 0 and eps = 0, a NaN, an
    infinity."""
    n = 256
    g = np.linspace(0.5, 2, n).astype(np.float32)
    x = np.random.default_rng(3).standard_normal((4, n)).astype(np.float32)
    x[0] = 0
    x[1, 17] = np.nan
    x[2, 200] = np.inf
    announce("rms_norm edge rows")
    for eps in (1e-6, 0.0):
        assert_same(host(S.rms_norm(dev(x), dev(g), eps, 4)), o.rms_norm(x, g, eps), f"eps {eps}")


def head_weights(S, ty, seed):
    rs = np.random.default_rng(seed)
    if ty == o.Q4_K:
        w = random_q4k(rs, VOCAB, HIDDEN)
    else:
        nb = VOCAB * HIDDEN // 32
        w = np.frombuffer(rs.bytes(nb * 34), np.uint8).reshape(nb, 34).copy()
        h = ((rs.integers(5, 10, nb, dtype=np.uint16) << 10) | rs.integers(0, 1024, nb, dtype=np.uint16))
        w[:, 0:2] = h.astype(np.uint16).view(np.uint8).reshape(nb, 2)
        w = w.ravel()
    return w


@pytest.mark.parametrize("ty,layout,rows", [(o.Q4_K, 0, 1), (o.Q4_K, 1, 1), (o.Q4_K, 0, 3), (o.Q4_K, 1, 64),
                                            (o.Q8_0, 0, 2), (o.Q8_0, 2, 1), (o.Q8_0, 2, 5)])
def test_logits_vocab_head(S, ty, layout, rows):
    """A 128256 x 4096 head: one decode row on the GEMV kernels (Q4_K in both layouts; Q8_0 SPLIT
    in one launch that quantizes the row in LDS), a few rows, and 64 rows on the matrix-core GEMM
    (X8)."""
    w = head_weights(S, ty, 0x10 + ty)
    rs = np.random.default_rng(rows)
    x = (rs.standard_normal((rows, HIDDEN)) * 3).astype(np.float32)
    g = (1 + 0.1 * rs.standard_normal(HIDDEN)).astype(np.float32)
    want = o.logits(ty, w, VOCAB, HIDDEN, g, 1e-5, x, rows, threads=16)
    wty = {o.Q4_K: S.WeightType.Q4K, o.Q8_0: S.WeightType.Q8_0}[ty]
    W = S.Weights(wty, dev(w), VOCAB, HIDDEN)
    if layout:
        W = S.repack(W, layout)
    announce(f"logits head {VOCAB}x{HIDDEN} ty={ty} layout={layout} rows={rows}")
    got = host(S.logits(W, dev(g), 1e-5, dev(x), rows))
    assert_same(got, want, "logits")


def test_logits_through_the_provider():
    """The Logits key with the head and the norm weight (weight 1) and eps (an F32 constant):
    the reference's op; with the head alone, the product of the already-normalised input (the
    graph's RmsNorm -> Logits)."""
    c = Ctx()
    try:
        P, pr = c.P, c.pr
        vocab, hidden, rows = 5000, 2048, 3
        rs = np.random.default_rng(41)
        w = random_q4k(rs, vocab, hidden)
        x = (rs.standard_normal((rows, hidden)) * 2).astype(np.float32)
        g = (1 + 0.1 * rs.standard_normal(hidden)).astype(np.float32)
        eps = np.float32(1e-6)
        key = {"op": "Logits", "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}], "layout": 0,
               "variant": 0}
        op = pr.prepare(c.ctx, key, shape(rows, vocab, hidden))
        wd, gd = dev(w), dev(g)
        xb, yb = c.put(x), c.empty(4 * rows * vocab)
        x_arg, y_arg = P.packed(xb, P.DT_F32, [rows, hidden]), P.packed(yb, P.DT_F32, [rows, vocab])
        announce("provider logits with its norm")
        eps_bits = int(np.array([eps], np.float32).view(np.uint32)[0])
        pr.launch(c.ctx, c.s, op, P.op_args([x_arg], [y_arg], [P.view(wd.data_ptr(), w.nbytes),
                                                               P.view(gd.data_ptr(), g.nbytes)],
                                            c.workspace(op), [P.Scalar(0, eps_bits)]))
        assert_same(c.get(yb, np.float32, (rows, vocab)), o.logits(o.Q4_K, w, vocab, hidden, g, eps, x, rows, 8),
                    "logits with norm")
        announce("provider logits head only")
        pr.launch(c.ctx, c.s, op, P.op_args([x_arg], [y_arg], [P.view(wd.data_ptr(), w.nbytes)], c.workspace(op)))
        assert_same(c.get(yb, np.float32, (rows, vocab)), o.gemv(o.Q4_K, w, vocab, hidden, x, rows, 8), "head only")
        with pytest.raises(P.ProviderError):  # a norm without its eps
            pr.launch(c.ctx, c.s, op, P.op_args([x_arg], [y_arg], [P.view(wd.data_ptr(), w.nbytes),
                                                                   P.view(gd.data_ptr(), g.nbytes)],
                                                c.workspace(op)))
    finally:
        c.close()
