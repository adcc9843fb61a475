"""The X8 weight layout (each run of eight Q4_K super-blocks stored chunk-major): the device and
host repacks agree with the definition and invert exactly, and the decode kernel and the GEMM
over repacked weights give the source layout's outputs bit for bit (the oracle's values)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_gemm import random_q4k

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


def x8_numpy(b: np.ndarray) -> np.ndarray:
    """The layout's definition on host bytes: chunk q of block i of a run of m at 16 (q m + i)."""
    nblk = b.size // 144
    out = np.empty_like(b)
    for g0 in range(0, nblk, 8):
        m = min(8, nblk - g0)
        run = b[g0 * 144:(g0 + m) * 144].reshape(m, 9, 16)
        out[g0 * 144:(g0 + m) * 144] = run.transpose(1, 0, 2).reshape(-1)
    return out


@pytest.mark.parametrize("nblk", [8, 16, 13, 1, 7, 8 * 57 + 5])
def test_repack_matches_definition_and_inverts(S, nblk):
    rs = np.random.default_rng(nblk)
    b = rs.integers(0, 256, nblk * 144, dtype=np.uint8)
    W = S.Weights(S.WeightType.Q4K, dev(b), nblk, 256)
    announce(f"x8 repack {nblk} blocks")
    r = S.repack(W)
    got = host(r.bytes)
    assert (got == x8_numpy(b)).all()
    back = torch.empty_like(r.bytes)
    S.lib().syn_q4k_repack(1, r.bytes.data_ptr(), back.data_ptr(), r.bytes.numel(), 1, None)
    assert (host(back) == b).all()
    h = np.empty_like(b)
    assert S.lib().syn_q4k_repack_host(1, b.ctypes.data, h.ctypes.data, b.size, 0) == 0
    assert (h == got).all()


@pytest.mark.parametrize("n_out,k", [(256, 4096), (96, 14336), (37, 3072), (50, 1536), (9, 16384), (5, 256)])
def test_decode_x8_equals_oracle(S, n_out, k):
    rs = np.random.default_rng(n_out + k)
    w = random_q4k(rs, n_out, k)
    x = o.normal(0xD0 + k, 1.0, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), n_out, k))
    announce(f"decode x8 {n_out}x{k}")
    got = host(S.gemv(W, dev(x), 1))
    assert_same(got, o.gemv(o.Q4_K, w, n_out, k, x, 1, threads=8), "x8 decode")


def test_batch_x8_equals_source_layout(S):
    shapes = [(6144, 4096), (4096, 4096), (1000, 14336), (37, 3072), (256, 1536)]
    rs = np.random.default_rng(3)
    Ws, Xs, Y0, Y1, W8 = [], [], [], [], []
    for n, k in shapes:
        w = S.Weights(S.WeightType.Q4K, dev(random_q4k(rs, n, k)), n, k)
        Ws.append(w)
        W8.append(S.repack(w))
        Xs.append(dev(o.normal(n + k, 1.0, k)))
        Y0.append(torch.empty(n, device="cuda"))
        Y1.append(torch.full((n,), float("nan"), device="cuda"))
    announce("batch x8 vs source")
    S.GemvBatch(Ws, Xs, Y0)()
    S.GemvBatch(W8, Xs, Y1)()
    for a, b in zip(Y0, Y1):
        assert_same(host(b), host(a), "x8 batch")


def test_batch_layer_full_shapes_equal_oracle(S):
    """The grouped decode launch over a whole Q4_K decode layer at Llama-3-8B shapes (QKV 6144x4096,
    O 4096x4096, gate and up 14336x4096, down 4096x14336), every output row, in both weight
    layouts, against the oracle."""
    shapes = [(6144, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336)]
    rs = np.random.default_rng(0x51A1)
    src, x8, xs, want = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        w = random_q4k(rs, n, k)
        x = o.normal(0x51A20003 + i, 1.0, k)
        want.append(o.gemv(o.Q4_K, w, n, k, x, 1, threads=16))
        W = S.Weights(S.WeightType.Q4K, dev(w), n, k)
        src.append(W)
        x8.append(S.repack(W))
        xs.append(dev(x))
    for name, ws in (("source", src), ("x8", x8)):
        ys = [torch.full((n,), float("nan"), device="cuda") for n, _ in shapes]
        announce(f"batch layer full shapes {name}")
        batch = S.GemvBatch(ws, xs, ys)
        for rep in range(2):
            batch()
            for i, y in enumerate(ys):
                assert_same(host(y), want[i], f"{name} problem {i} rep {rep}")


def _batch_case(S, shapes, seed):
    rs = np.random.default_rng(seed)
    ws, xs, ys, raw = [], [], [], []
    for n, k in shapes:
        w = random_q4k(rs, n, k)
        raw.append(w)
        ws.append(S.repack(S.Weights(S.WeightType.Q4K, dev(w), n, k)))
        xs.append(torch.empty(k, device="cuda"))
        ys.append(torch.full((n,), float("nan"), device="cuda"))
    return ws, xs, ys, raw


def _set_rows(shapes, xs, seed):
    vals = []
    for i, (n, k) in enumerate(shapes):
        x = o.normal(seed + i, 1.0, k)
        xs[i].copy_(dev(x))
        vals.append(x)
    torch.cuda.synchronize()
    return vals


def test_batch_x8_new_rows_each_call(S):
    """One workspace, six calls with new rows each: every call equals the oracle (nothing of an
    earlier call's quantized rows stands in for the next call's)."""
    shapes = [(512, 4096), (300, 14336), (64, 2048)]
    ws, xs, ys, raw = _batch_case(S, shapes, 0x5180)
    batch = S.GemvBatch(ws, xs, ys)
    for call_no in range(6):
        x = _set_rows(shapes, xs, 0x5190 + 10 * call_no)
        announce(f"batch call {call_no}")
        batch()
        for i, (n, k) in enumerate(shapes):
            assert_same(host(ys[i]), o.gemv(o.Q4_K, raw[i], n, k, x[i], 1, threads=16), f"call {call_no} problem {i}")


def test_batch_x8_captured_replays_equal_oracle(S):
    """The grouped decode captured into a graph: replays with new rows, eager work and
    synchronizations between them, each equal the oracle."""
    shapes = [(640, 4096), (96, 14336)]
    ws, xs, ys, raw = _batch_case(S, shapes, 0x51A0)
    batch = S.GemvBatch(ws, xs, ys)
    _set_rows(shapes, xs, 0x51B0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        batch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        batch()
    for rep in range(3):
        x = _set_rows(shapes, xs, 0x51C0 + 10 * rep)
        announce(f"batch captured replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        for i, (n, k) in enumerate(shapes):
            assert_same(host(ys[i]), o.gemv(o.Q4_K, raw[i], n, k, x[i], 1, threads=16), f"replay {rep} problem {i}")


@pytest.mark.parametrize("rows,n_out,k", [(32, 64, 2048), (64, 300, 4096), (100, 256, 14336)])
def test_gemm_x8_equals_oracle(S, rows, n_out, k):
    rs = np.random.default_rng(rows + n_out + k)
    w = random_q4k(rs, n_out, k)
    x = o.normal(0xE0 + rows, 1.0, rows * k).reshape(rows, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), n_out, k))
    announce(f"gemm x8 rows={rows} {n_out}x{k}")
    got = host(S.gemv(W, dev(x), rows))
    assert_same(got, o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8), "x8 gemm")


@pytest.mark.parametrize("rows,n_out,k", [(2, 14336, 4096), (3, 14336, 4096), (8, 4096, 14336), (7, 37, 1536),
                                          (4, 9, 16384), (5, 300, 256), (16, 8192, 4096), (17, 1000, 2304),
                                          (31, 33, 1536), (13, 4096, 14336), (2, 37, 1536), (2, 4096, 14336),
                                          (2, 9, 16384), (3, 8200, 2304), (3, 4096, 4096), (3, 6144, 4096),
                                          (3, 37, 1536), (3, 300, 14336), (4, 14336, 4096), (4, 6144, 4096),
                                          (4, 37, 1536), (4, 300, 2304), (2, 300, 8192)])
def test_x8_rows_2_to_31_equal_oracle(S, rows, n_out, k):
    """2..31 rows over X8 weights: at two rows, and three or four of at most 16 super-blocks, the
    decode kernel with the rows side by side in LDS (16, 32 or 64 lanes a row, lanes past the
    row's blocks, a partial last workgroup, one fold lane per weight row and activation row; up
    to 16 super-blocks the rows quantized in its workgroups); otherwise the decode expert kernel:
    the rows quantized once,
    four-row groups on the int8 matrix cores, 16- or 32-row items (k need not be a multiple of
    2048: the X8 chunk addresses are computed per super-block)."""
    rs = np.random.default_rng(rows * 7 + n_out + k)
    w = random_q4k(rs, n_out, k)
    x = o.normal(0xF0 + rows, 1.0, rows * k).reshape(rows, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), n_out, k))
    announce(f"x8 rows={rows} {n_out}x{k}")
    got = host(S.gemv(W, dev(x), rows))
    assert_same(got, o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=16), "x8 rows")


@pytest.mark.parametrize("n_out,k", [(14336, 4096), (4096 + 9, 2048), (37, 4096), (16 * 257 + 3, 4096),
                                     (16 * 512, 2048)])
def test_x8_rows_whole_runs_equal_oracle(S, n_out, k):
    """2 to 8 rows over X8 rows of whole 8-block runs: the decode kernel with the rows quantized in
    its workgroups (2 and 3 rows) and the quantization launch then the line-order expert kernel
    (5, 7, 8 rows), at one and two runs a row, a partial last 16-row group, and thousands of row
    groups."""
    rs = np.random.default_rng(n_out * 3 + k)
    w = random_q4k(rs, n_out, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), n_out, k))
    for rows in (2, 3, 5, 7, 8):
        x = o.normal(0xF1 + rows + n_out, 1.0, rows * k).reshape(rows, k)
        announce(f"x8 whole-run rows={rows} {n_out}x{k}")
        y = torch.full((rows, n_out), float("nan"), device="cuda")
        S.gemv(W, dev(x), rows, y=y)
        assert_same(host(y), o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=16), f"x8 whole-run rows {rows}")


def test_x8_refusals(S):
    W = S.repack(S.Weights(S.WeightType.Q4K, torch.zeros(64 * 6 * 144, dtype=torch.uint8, device="cuda"), 64, 1536))
    x = torch.zeros(32, 1536, device="cuda")
    with pytest.raises(S.SynError):  # from 32 rows the GEMM takes rows of whole 8-block runs only
        S.gemv(W, x, 32)


@pytest.mark.parametrize("rows,n_out,k", [(2, 14336, 4096), (8, 4096, 14336), (9, 300, 1536), (31, 37, 256),
                                          (20, 6144, 4096)])
def test_source_q4k_rows_2_to_31_equal_oracle(S, rows, n_out, k):
    """The same kernel over GGUF-order Q4_K weights (syn_gemv)."""
    rs = np.random.default_rng(rows * 11 + n_out + k)
    w = random_q4k(rs, n_out, k)
    x = o.normal(0xF8 + rows, 1.0, rows * k).reshape(rows, k)
    W = S.Weights(S.WeightType.Q4K, dev(w), n_out, k)
    announce(f"source q4k rows={rows} {n_out}x{k}")
    y = torch.full((rows, n_out), float("nan"), device="cuda")
    S.gemv(W, dev(x), rows, y=y)
    assert_same(host(y), o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=16), "source rows")
