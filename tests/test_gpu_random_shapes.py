"""Gemv over seeded random shapes: weight type, source or repacked layout, row count, matrix rows
and row length drawn from a fixed seed per case, every output bit-identical to the oracle.

The library picks among its one-row, few-row, split, staged, K-split and prefill kernels by shape
and by cost estimates fitted on timings; every choice computes the same bits, so a mismatch at
any of those boundaries is a fault of the kernel chosen there.  The fixed-shape tests pin each
kernel at the shapes it was written for; these cases land between them."""
import numpy as np
import pytest

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_gemm import random_q4k

pytestmark = pytest.mark.gpu

ROWS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 13, 16, 17, 24, 31, 32, 33, 48, 64, 65, 100]
TYPES = [o.Q4_0, o.Q8_0, o.Q4_K, o.F16, o.BF16]
MAX_WEIGHTS = 12 << 20  # elements a case's matrix holds at most


def draw(case: int):
    """(type, repacked, rows, n_out, k) of one case."""
    rs = np.random.default_rng(0x5A7D00 + case)
    ty = TYPES[case % len(TYPES)]
    repacked = ty in (o.Q4_0, o.Q8_0, o.Q4_K) and bool(rs.integers(0, 2))
    rows = int(rs.choice(ROWS))
    be = o.BLOCK_ELEMS[ty]
    if ty == o.Q4_K and repacked and rows >= 32:
        k = 2048 * int(rs.integers(1, 8))  # the X8 GEMM takes rows of whole 8-block runs
    elif ty in (o.F16, o.BF16):
        k = int(rs.integers(1, 9000))
    else:
        k = be * int(rs.integers(1, 16384 // be + 1))
    n_out = int(rs.integers(1, max(2, min(6000, MAX_WEIGHTS // k)) + 1))
    return ty, repacked, rows, n_out, k


def weights(rs, ty, n_out, k):
    """GGUF bytes: random Q4_K blocks, ggml's Q4_0 / Q8_0 of N(0, 0.02), F16 of N(0, 0.02), BF16
    of it rounded to nearest even."""
    if ty == o.Q4_K:
        return random_q4k(rs, n_out, k)
    v = rs.normal(0.0, 0.02, n_out * k).astype(np.float32)
    if ty in (o.Q4_0, o.Q8_0):
        return o.quantize(ty, v)
    if ty == o.F16:
        return v.astype(np.float16).view(np.uint8)
    b = v.view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


@pytest.mark.parametrize("case", range(200))
def test_random_shape_equals_oracle(S, case):
    ty, repacked, rows, n_out, k = draw(case)
    rs = np.random.default_rng(0x5A7E00 + case)
    w = weights(rs, ty, n_out, k)
    x = o.normal(0x5A7F00 + case, 1.0, rows * k)
    W = S.Weights(S.WeightType(ty), dev(w), n_out, k)
    if repacked:
        W = S.repack(W)
    announce(f"random case {case}: ty={ty} repacked={repacked} rows={rows} {n_out}x{k}")
    got = host(S.gemv(W, dev(x.reshape(rows, k)), rows))
    assert_same(got, o.gemv(ty, w, n_out, k, x, rows, threads=16), f"case {case}")
