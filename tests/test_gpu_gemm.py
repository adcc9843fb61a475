"""GPU parity of the prefill Q4_K GEMM (the matrix-core path Gemv takes at 32 rows or more)
against the CPU oracle: every output bit-identical to the Gemv value
(crates/kernels-cpu/src/gemv.rs:435-547)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


def random_q4k(rs, n_out, k, lo_exp=5, hi_exp=10):
    """Random Q4_K blocks: every code, 6-bit scale and minimum pattern; F16 d and dmin with biased
    exponents lo_exp..hi_exp-1."""
    nb = n_out * k // 256
    b = rs.integers(0, 256, (nb, 144), dtype=np.uint8)
    h = ((rs.integers(lo_exp, hi_exp, (nb, 2), dtype=np.uint16) << 10)
         | rs.integers(0, 1024, (nb, 2), dtype=np.uint16)).astype(np.uint16)
    b[:, 0:4] = h.view(np.uint8).reshape(nb, 4)
    return b.ravel()


def run_both(S, w, n_out, k, x, rows):
    """(the Gemv op, the split GEMM entries) on the same operands."""
    W = S.Weights(S.WeightType.Q4K, dev(w), n_out, k)
    xd = dev(x.astype(np.float32))
    y1 = host(S.gemv(W, xd, rows))
    ws = S.gemm_workspace(rows, k)
    S.gemm_quantize_into(xd, rows, k, ws)
    y2 = torch.full((rows, n_out), float("nan"), device="cuda")
    S.gemm_quantized(W, ws, rows, y2)
    return y1, host(y2)


@pytest.mark.parametrize("rows,n_out,k", [(32, 256, 256), (64, 512, 1024), (65, 300, 512),
                                          (100, 1000, 2048), (130, 256, 4096), (40, 64, 768),
                                          (33, 17, 256), (200, 520, 1536)])
def test_gemm_equals_oracle(S, rows, n_out, k):
    rs = np.random.default_rng(rows * 1000 + n_out + k)
    w = random_q4k(rs, n_out, k)
    x = o.normal(0x6E11 + rows + k, 1.0, rows * k).reshape(rows, k)
    announce(f"gemm rows={rows} n_out={n_out} k={k}")
    y1, y2 = run_both(S, w, n_out, k, x, rows)
    want = o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8)
    assert_same(y1, want, "gemv op")
    assert_same(y2, want, "split gemm")


def test_gemm_extreme_magnitudes(S):
    """Scales 63 and codes 15 against codes +-127 of one sign: the largest sums the exact F16
    accumulation has to carry (256 * 127 * 512 < 2^24), and the smallest (codes 0)."""
    rows, n_out, k = 64, 64, 1024
    rs = np.random.default_rng(11)
    w = random_q4k(rs, n_out, k).reshape(-1, 144)
    w[:, 4:16] = 0xFF          # every 6-bit scale and minimum 63
    w[0::3, 16:] = 0xFF        # codes 15
    w[1::3, 16:] = 0x00        # codes 0
    w[2::3, 16:] = 0xF0        # alternating 0 / 15
    w = w.ravel()
    x = np.abs(o.normal(5, 1.0, rows * k)).reshape(rows, k) + 1.0
    x[1::2] *= -1.0            # every code +127 or -127 region by region
    x[5] = 3.0                 # one flat row: every code 127
    announce("gemm extreme magnitudes")
    y1, y2 = run_both(S, w, n_out, k, x, rows)
    want = o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8)
    assert_same(y1, want, "gemv op")
    assert_same(y2, want, "split gemm")


def test_gemm_nonfinite_and_zero_blocks(S):
    rows, n_out, k = 48, 128, 768
    rs = np.random.default_rng(12)
    w = random_q4k(rs, n_out, k)
    x = o.normal(13, 1.0, rows * k).reshape(rows, k)
    x[3, 7] = np.nan
    x[9, 300] = np.inf
    x[17, 256:512] = 0.0
    x[20, :] = 0.0
    x[30, 600] = -1e-39
    announce("gemm nonfinite and zero blocks")
    y1, y2 = run_both(S, w, n_out, k, x, rows)
    want = o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8)
    assert_same(y1, want, "gemv op")
    assert_same(y2, want, "split gemm")


def test_gemm_wide_scale_range(S):
    """d and dmin across the F16 range (subnormal to large) so the terms span many exponents."""
    rows, n_out, k = 40, 96, 512
    rs = np.random.default_rng(14)
    w = random_q4k(rs, n_out, k, lo_exp=0, hi_exp=30)
    x = o.normal(15, 3.0, rows * k).reshape(rows, k)
    announce("gemm wide scale range")
    y1, y2 = run_both(S, w, n_out, k, x, rows)
    want = o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8)
    assert_same(y1, want, "gemv op")
    assert_same(y2, want, "split gemm")


@pytest.mark.parametrize("n_out,k", [(14336, 4096), (4096, 14336)])
def test_gemm_prefill_config_shapes(S, n_out, k):
    """The dense prefill shapes at 2048 tokens (X N(0,1) rounded to BF16 values): the GEMM equals
    the oracle on the whole output, and so does the row-group GEMV path."""
    rows = 2048
    rs = np.random.default_rng(n_out + k)
    w = random_q4k(rs, n_out, k)
    xf = torch.from_numpy(o.normal(0x51A20005, 1.0, rows * k)).to(torch.bfloat16).to(torch.float32)
    x = xf.numpy().reshape(rows, k)
    W = S.Weights(S.WeightType.Q4K, dev(w), n_out, k)
    xd = dev(x)
    announce(f"gemm prefill shape {n_out}x{k} rows {rows}")
    ws = S.gemm_workspace(rows, k)
    S.gemm_quantize_into(xd, rows, k, ws)
    y = torch.empty(rows, n_out, device="cuda")
    S.gemm_quantized(W, ws, rows, y)
    # the row-group GEMV kernel on the same rows (act layout of syn_act_quantize)
    ws2 = S.new_workspace(S.WeightType.Q4K, rows, k)
    S.quantize_into(S.WeightType.Q4K, xd, rows, k, ws2)
    y2 = torch.empty(rows, n_out, device="cuda")
    S.gemv_quantized(W, ws2, rows, y2)
    want = o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=16)
    assert_same(host(y), want, "gemm vs oracle")
    assert_same(host(y2), want, "row-group gemv vs oracle")
