"""The SPLIT weight layout of Q8_0 and Q4_0 matrices (every block's codes, then every block's F16
scale): the device repack is its definition and inverts exactly, and the split decode kernel
(1 to 8 rows, eight at a time beyond) and the int8 matrix-core GEMM (Q8_0, 9 rows or more) give
the oracle's Gemv values bit for bit (crates/kernels-cpu/src/gemv.rs:435-492)."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from refgen import GemvRng, gemv_activations, gemv_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


WT = {o.Q8_0: "Q8_0", o.Q4_0: "Q4_0"}


def split_numpy(b, bb):
    blocks = b.reshape(-1, bb)
    return np.concatenate([blocks[:, 2:].ravel(), blocks[:, :2].ravel()])


@pytest.mark.parametrize("ty,bb", [(o.Q8_0, 34), (o.Q4_0, 18)])
@pytest.mark.parametrize("nblk", [1, 255, 256, 257, 4096 + 3])
def test_split_repack_matches_definition_and_inverts(S, ty, bb, nblk):
    rs = np.random.default_rng(nblk * ty)
    b = rs.integers(0, 256, nblk * bb, dtype=np.uint8)
    W = S.Weights(S.WeightType(ty), dev(b), nblk, 32)
    announce(f"split repack ty={ty} {nblk} blocks")
    r = S.repack(W)
    assert r.layout == S.LAYOUT_SPLIT
    got = host(r.bytes)
    assert (got == split_numpy(b, bb)).all()
    back = torch.empty_like(r.bytes)
    assert S.lib().syn_split_repack(2, ty, r.bytes.data_ptr(), back.data_ptr(), r.bytes.numel(), 1, None) == 0
    torch.cuda.synchronize()
    assert (host(back) == b).all()


def check(S, ty, n_out, k, rows, seed, w=None):
    rng = GemvRng(seed)
    if w is None:
        w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    W = S.repack(S.Weights(S.WeightType(ty), dev(w), n_out, k))
    announce(f"split gemv {WT[ty]} {n_out}x{k} rows={rows}")
    y = torch.full((rows, n_out), float("nan"), device="cuda")
    S.gemv(W, dev(x.astype(np.float32)), rows, y=y)
    want = o.gemv(ty, w, n_out, k, x, rows, threads=8)
    assert_same(host(y), want, f"{WT[ty]} {n_out}x{k} rows {rows}")
    if rows in (1, 9):  # the product alone over rows quantized beforehand
        ws = S.new_workspace(S.WeightType(ty), rows, k)
        S.quantize_into(S.WeightType(ty), dev(x.astype(np.float32)), rows, k, ws)
        y.fill_(float("nan"))
        S.gemv_quantized(W, ws, rows, y)
        assert_same(host(y), want, f"{WT[ty]} quantized rows {rows}")
    return w


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
@pytest.mark.parametrize("n_out,k", [(37, 32), (300, 1024), (41, 3072), (9, 14336), (130, 16384 + 32), (9, 45056)])
def test_split_decode_rows_equal_oracle(S, ty, n_out, k):
    """1 to 8 rows (staged activations for narrow rows, global reads for wide ones), 9 and 20 rows
    (eight-row groups, or the GEMM where it is the faster); row lengths of 1 to 1408 blocks,
    partial last load groups and row counts not multiples of eight.  One row is one launch that
    quantizes its row in LDS up to 39,296 (Q4_0) or 43,680 (Q8_0) values; 45,056 takes the
    quantization launch first."""
    w = None
    for rows in (1, 2, 3, 5, 8, 9, 20):
        w = check(S, ty, n_out, k, rows, 1000 * rows + n_out + k + ty, w)


@pytest.mark.parametrize("ty,n_out,k,rowss", [
    (o.Q8_0, 14336, 4096, [1, 8, 32, 128]),  # Q8_0 decode and prefill of the 14336 x 4096 matrix
    (o.Q4_0, 4096, 4096, [1, 4, 32, 128]),   # the Q4_0 4096 x 4096 decode and a few rows
])
def test_split_config_shapes_equal_oracle(S, ty, n_out, k, rowss):
    x = o.normal(0x5E11 + k, 0.02, n_out * k)
    w = o.quantize(ty, x)
    for rows in rowss:
        check(S, ty, n_out, k, rows, 0x5E12 + rows, w)


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
@pytest.mark.parametrize("n_out,k", [(4096 + 37, 1024), (4096 + 5, 14336 + 32), (2048 + 9, 4096)])
def test_split_one_row_workgroup_fold_equal_oracle(S, ty, n_out, k):
    """One row quantized in the product's workgroups, whose rows are folded together: workgroups
    of sixteen rows (Q4_0 at 4096 rows or more) and of eight, the last one partly past the
    matrix; rows of one to four 128-block fold chunks, the last one partial."""
    w = o.quantize(ty, o.normal(0x5E21 + n_out + k, 0.02, n_out * k))
    check(S, ty, n_out, k, 1, 0x5E22 + n_out, w)


def test_split_gemm_edges_equal_oracle(S):
    """The GEMM's clamped tiles: weight rows not multiples of 16 (or 64), token counts not
    multiples of 32, one-block rows, many tiles of tokens."""
    for n_out, k, rows in ((1, 32, 9), (17, 64, 33), (63, 96, 31), (65, 256, 100), (200, 2048, 257)):
        check(S, o.Q8_0, n_out, k, rows, n_out * 31 + rows)


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
def test_split_gemm_staged_shapes_equal_oracle(S, ty):
    """The LDS-staged GEMMs: the K-split form (up to 16 tokens, rows of whole 16-block stages:
    9 and 16 rows here) and the staged form (more tokens, or rows of whole 4-block stages: every
    token-tile variant, 16, 32 and 64 tokens a workgroup, one or two 16-token tiles a wavefront),
    partial workgroups of rows and tokens, one stage and many; for Q4_0 (64-byte row lines,
    nibbles widened in registers) and Q8_0."""
    w = None
    for rows in (9, 16, 17, 31, 32, 33, 64, 65, 127):
        w = check(S, ty, 50, 512, rows, 7000 + rows + ty, w)
    # the last three launch enough wavefronts for two-tile wavefronts (32 and 64 tokens)
    # (160, 14336, 24): the K-split form over two token tiles at long rows
    for n_out, k, rows in ((33, 128, 40), (96, 4096, 48), (1, 128, 70), (4097, 256, 5), (160, 14336, 24),
                           (32800, 128, 20), (32770, 128, 31), (4096, 256, 300)):
        check(S, ty, n_out, k, rows, n_out + k + rows + ty)


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
def test_split_gemm_few_rows_equal_oracle(S, ty):
    """2 to 16 rows over 14336-row matrices, where the staged GEMM (one 16-token tile; at this
    many rows it is estimated faster than the K-split form) takes over from the split decode
    kernel at a few rows: full tiles, a partial last row tile and a partial last row group."""
    x = o.normal(0xF3 + ty, 0.02, 14336 * 4096)
    w = o.quantize(ty, x)
    for rows in (2, 5, 8, 13, 16):
        check(S, ty, 14336, 4096, rows, 0xF30 + rows + ty, w)
    cb = 34 if ty == o.Q8_0 else 18
    check(S, ty, 14329, 4096, 7, 0xF31 + ty, w[:14329 * 128 * cb])


def test_split_q4_0_extreme_codes_equal_oracle(S):
    """Q4_0 codes 0 and 15 (n - 8 = -8 and 7) against activation codes of +-127 in every block:
    the widened nibbles at both ends, whose exact block sums are as large as Q4_0 makes them."""
    n_out, k = 64, 1024
    nb = k // 32
    rng = np.random.default_rng(0x40E)
    w = np.zeros((n_out * nb, 18), np.uint8)
    w[:, 0:2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
    w[:, 2:] = rng.choice(np.array([0x00, 0xFF, 0x0F, 0xF0], np.uint8), size=(n_out * nb, 16))
    w = w.reshape(-1)
    for rows in (2, 20, 70):
        x = np.where(rng.random(rows * k) < 0.5, -1.0, 1.0).astype(np.float32)
        W = S.repack(S.Weights(S.WeightType(o.Q4_0), dev(w), n_out, k))
        announce(f"split gemv Q4_0 extreme codes {n_out}x{k} rows={rows}")
        y = torch.full((rows, n_out), float("nan"), device="cuda")
        S.gemv(W, dev(x), rows, y=y)
        want = o.gemv(o.Q4_0, w, n_out, k, x, rows, threads=8)
        assert_same(host(y), want, f"Q4_0 extreme codes rows {rows}")


# F16 weight scales across the range: subnormal (both signs), the largest finite, zeros of both
# signs, ones, and ordinary values; the products dw * dx then run from subnormal F32 to large
SCALE_BITS = np.array([0x0001, 0x0200, 0x03FF, 0x8001, 0x83FF, 0x7BFF, 0xFBFF, 0x0000, 0x8000,
                       0x3C00, 0xBC00, 0x2E66, 0x1400, 0x0400, 0x5640, 0xD0F0], np.uint16)


@pytest.mark.parametrize("ty,bb", [(o.Q8_0, 34), (o.Q4_0, 18)])
@pytest.mark.parametrize("n_out,k", [(64, 2048), (300, 1024)])
def test_split_extreme_scales_equal_oracle(S, ty, bb, n_out, k):
    """Weights whose F16 scales span subnormals, the largest finite F16 and signed zeros,
    against activation blocks of magnitudes 1e-6 to 1e4, at one row (the workgroups' quantization,
    and the product on a quantized row) and at 2 to 128 rows (the split decode kernel, the int8
    matrix-core GEMMs): the scale products dw * dx from subnormal F16 operands, each rounded once
    as the reference rounds it."""
    nb = k // 32
    rng = np.random.default_rng(0x5CA1E + n_out + ty)
    w = rng.integers(0, 256, (n_out * nb, bb), dtype=np.uint8)
    sc = rng.choice(SCALE_BITS, size=n_out * nb)
    w[:, 0] = (sc & 0xFF).astype(np.uint8)
    w[:, 1] = (sc >> 8).astype(np.uint8)
    w = w.reshape(-1)
    W = S.repack(S.Weights(S.WeightType(ty), dev(w), n_out, k))
    for rows in (1, 2, 8, 16, 32, 128):
        # a magnitude per 32-value block, 1e-6 to 1e4: activation scales from F16 subnormals up
        mag = np.repeat(np.float32(10.0) ** rng.integers(-6, 5, rows * k // 32).astype(np.float32), 32)
        x = (rng.standard_normal(rows * k).astype(np.float32) * mag).astype(np.float32)
        announce(f"split gemv {WT[ty]} extreme scales {n_out}x{k} rows={rows}")
        y = torch.full((rows, n_out), float("nan"), device="cuda")
        S.gemv(W, dev(x), rows, y=y)
        want = o.gemv(ty, w, n_out, k, x, rows, threads=8)
        assert_same(host(y), want, f"{WT[ty]} extreme scales rows {rows}")
        if rows in (1, 8, 32):
            ws = S.new_workspace(S.WeightType(ty), rows, k)
            S.quantize_into(S.WeightType(ty), dev(x), rows, k, ws)
            y.fill_(float("nan"))
            S.gemv_quantized(W, ws, rows, y)
            assert_same(host(y), want, f"{WT[ty]} extreme scales quantized rows {rows}")


@pytest.mark.parametrize("ty,n_out,k,layout,ok", [
    (o.Q8_0, 64, 512, 2, False),   # SPLIT: the scale section sits after every block's codes
    (o.Q4_0, 64, 512, 2, False),
    (o.Q4_K, 3, 256, 1, False),    # X8 with a final run of 3 super-blocks
    (o.Q4_K, 16, 512, 1, True)])   # X8 in whole runs of 8: a longer view reads the same bytes
def test_repacked_view_longer_than_the_matrix(S, ty, n_out, k, layout, ok):
    """A repacked view must be the repack of its matrix alone where the layout places bytes by the
    total length; a longer view is refused before anything runs (or, in whole X8 runs, computes the
    same values)."""
    rng = GemvRng(4242 + ty)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, 2, k).astype(np.float32)
    W = S.repack(S.Weights(S.WeightType(ty), dev(w), n_out, k))
    assert W.layout == layout
    longer = torch.zeros(W.bytes.numel() + 256, dtype=torch.uint8, device="cuda")
    longer[:W.bytes.numel()] = W.bytes
    y = torch.full((2, n_out), float("nan"), device="cuda")
    need = C.c_uint64(0)
    assert S.lib().syn_gemv_layout_workspace_bytes(layout, ty, 2, k, C.byref(need)) == 0
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device="cuda")
    announce(f"longer view ty={ty} {n_out}x{k} layout={layout}")
    args = (layout, ty, longer.data_ptr(), longer.numel(), n_out, k, dev(x).data_ptr(), 2, y.data_ptr(),
            ws.data_ptr(), ws.numel(), None)
    rc = S.lib().syn_gemv_layout(*args)
    if ok:
        assert rc == 0
        assert_same(host(y), o.gemv(ty, w, n_out, k, x, 2), "whole X8 runs")
    else:
        assert rc != 0 and b"repack of the matrix alone" in S.lib().syn_last_error()
        torch.cuda.synchronize()
        assert torch.isnan(y).all()
