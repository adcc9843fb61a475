"""Pins of the oracle's RmsNorm and Logits (CPU only): crates/kernels/src/reference/norm.rs
(Norm::row and its documented edge cases) and crates/kernels/src/reference/linear.rs:118-161
(each row normalised, then the head).  Each check is computed without the oracle's code path,
and the operation-order case is one where the plausible other orders give other bits."""
import numpy as np
import pytest

from oracle import oracle as o

f32 = np.float32


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def spec_row(x, g, eps, order="xs_g"):
    """norm.rs:39-47 step by step in F32 (the sum of squares of 4 values is one sequential block);
    `order` plants the other groupings of the final product."""
    ss = f32(0)
    for v in x:
        ss = f32(ss + f32(v * v))
    mean = f32(ss / f32(len(x)))
    scale = f32(f32(1) / np.sqrt(f32(mean + eps)))
    if order == "xs_g":
        return ((x * scale).astype(f32) * g).astype(f32)
    if order == "xg_s":
        return ((x * g).astype(f32) * scale).astype(f32)
    return (x * (scale * g).astype(f32)).astype(f32)


def test_rms_norm_operation_order():
    """y = (x * scale) * g: on this row the groupings (x g) scale and x (scale g) round to
    other bits, so the oracle's agreement pins the order."""
    x = np.array([4.125, 5.0, 0.25, 5.0], f32)
    g = np.array([1.46875, 1.609375, 1.96875, 0.890625], f32)
    eps = f32(1e-5)
    want = spec_row(x, g, eps)
    assert not np.array_equal(bits(want), bits(spec_row(x, g, eps, "xg_s")))
    assert not np.array_equal(bits(want), bits(spec_row(x, g, eps, "x_sg")))
    assert np.array_equal(bits(o.rms_norm(x[None], g, eps)[0]), bits(want))


def test_rms_norm_exact_rows():
    """Rows whose mean square is a power of four: scale is an exact power of two, so y = x g / 2^k
    exactly, whatever the row length (and the sum of squares of equal terms is exact)."""
    for n, c in [(32, 2.0), (100, 0.5), (4096, 8.0), (7, 1.0)]:
        x = np.full((2, n), c, f32)
        x[1] *= -1
        g = np.linspace(-3, 3, n).astype(f32)
        y = o.rms_norm(x, g, 0.0)
        want = (x / f32(abs(c))) * g
        assert np.array_equal(bits(y), bits(want)), n


def test_rms_norm_edge_cases():
    """norm.rs module docs: zeros give zeros when eps > 0 and NaN when eps = 0; a NaN makes the
    row NaN; an infinity makes the row NaN where x is infinite and +-0 elsewhere."""
    g = np.arange(1, 9).astype(f32)
    z = np.zeros((1, 8), f32)
    assert np.array_equal(bits(o.rms_norm(z, g, 1e-6)), bits(z))
    assert np.isnan(o.rms_norm(z, g, 0.0)).all()
    x = np.arange(8, dtype=f32)[None] - 3
    xn = x.copy()
    xn[0, 5] = np.nan
    assert np.isnan(o.rms_norm(xn, g, 1e-6)).all()
    xi = x.copy()
    xi[0, 2] = np.inf
    y = o.rms_norm(xi, g, 1e-6)[0]
    assert np.isnan(y[2])
    rest = np.delete(y, 2)
    assert (rest == 0).all()
    assert (np.signbit(rest) == np.signbit(np.delete(x[0] * g, 2))).all()


def test_rms_norm_within_the_f64_bound():
    """Against the F64 value of the same definition: the sum of squares (n roundings at most),
    the division, the square root, the reciprocal and the two products; a norm that divides by
    n - 1 or drops eps misses it."""
    rs = np.random.default_rng(12)
    n = 4096
    x = (rs.standard_normal((8, n)) * 10.0 ** rs.integers(-2, 3, (8, 1))).astype(f32)
    g = (1 + rs.standard_normal(n) * 0.1).astype(f32)
    eps = f32(1e-5)
    y = o.rms_norm(x, g, eps).astype(np.float64)
    x64, g64 = x.astype(np.float64), g.astype(np.float64)
    ms = (x64 * x64).mean(axis=1, keepdims=True)
    want = x64 / np.sqrt(ms + float(eps)) * g64
    bound = (40 + 8) * 2.0 ** -24 * np.abs(want) + 1e-30
    assert (np.abs(y - want) <= bound).all()
    wrong = x64 / np.sqrt((x64 * x64).sum(axis=1, keepdims=True) / (n - 1) + float(eps)) * g64
    assert not (np.abs(wrong - want) <= bound).all()
    x_small = (rs.standard_normal((1, n)) * 1e-3).astype(f32)
    no_eps = x_small.astype(np.float64) / np.sqrt((x_small.astype(np.float64) ** 2).mean()) * g64
    with_eps = o.rms_norm(x_small, g, eps).astype(np.float64)
    assert not (np.abs(with_eps - no_eps) <= (48 * 2.0 ** -24) * np.abs(no_eps)).all()


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_K])
def test_logits_normalises_before_the_head(ty):
    """Rows whose normalisation is an exact halving (mean square 4, eps 0, g 1): Logits equals
    the head's Gemv of x / 2, and not of x; and a weight g of powers of two scales its own
    column only (the Gemv of (x / 2) g, exact)."""
    vocab, hidden, rows = 40, 512, 3
    rs = np.random.default_rng(ty)
    w = o.quantize(ty, (rs.standard_normal(vocab * hidden) * 0.02).astype(f32))
    x = np.where(rs.random((rows, hidden)) < 0.5, f32(2), f32(-2)).astype(f32)
    ones = np.ones(hidden, f32)
    y = o.logits(ty, w, vocab, hidden, ones, 0.0, x, rows)
    assert np.array_equal(bits(y), bits(o.gemv(ty, w, vocab, hidden, x / f32(2), rows)))
    assert not np.array_equal(bits(y), bits(o.gemv(ty, w, vocab, hidden, x, rows)))
    g = (2.0 ** rs.integers(-2, 3, hidden)).astype(f32)
    y2 = o.logits(ty, w, vocab, hidden, g, 0.0, x, rows)
    assert np.array_equal(bits(y2), bits(o.gemv(ty, w, vocab, hidden, (x / f32(2)) * g, rows)))
