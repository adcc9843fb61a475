"""GPU parity of the activation quantizers, the GEMV kernels and the weight packers against the
CPU oracle (itself pinned to the reference's golden outputs).  Bit-exact throughout."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, bits, dev, host, require_gpu
from oracle import oracle as o
from refgen import GemvRng, gemv_activations, gemv_weights, gemv_widths, quant_values

pytestmark = pytest.mark.gpu

QTYPES = [o.Q8_0, o.Q4_0, o.Q4_K]


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


def align(v, a=256):
    return (v + a - 1) // a * a


def read_act(ws, kind, rows, k):
    """Splits the device activation workspace (codes | scales | 32-sums, 256-byte sections)."""
    n = rows * k
    nd = n // 32 if kind == o.ACT_Q8_0 else n // 256
    d_off = align(n)
    s_off = align(d_off + 4 * nd)
    raw = host(ws)
    codes = raw[:n].view(np.int8)
    d = raw[d_off:d_off + 4 * nd].view(np.float32)
    sums = raw[s_off:s_off + 4 * (n // 32)].view(np.int32)
    return codes, d, sums


def gpu_gemv(S, ty, w, n_out, k, x, rows):
    W = S.Weights(ty, dev(w), n_out, k)
    y = S.gemv(W, dev(x.astype(np.float32)), rows)
    return host(y)


# ---- activation quantizers against the reference's golden vectors -------------------------
def test_act_quant_golden(S):
    from test_oracle_pins import ACT_CASES
    for case in ACT_CASES:
        x = case["in"]
        n = x.size
        if "q8_0 cpu" not in case:
            continue
        announce(f"act_quant golden {case['name']}")
        for ty, kind in ((S.WeightType.Q4_0, o.ACT_Q8_0), (S.WeightType.Q4K, o.ACT_Q8K)):
            if n % (256 if kind == o.ACT_Q8K else 32):
                continue
            ws = S.new_workspace(ty, 1, n)
            S.quantize_into(ty, dev(x), 1, n, ws)
            codes, d, sums = read_act(ws, kind, 1, n)
            wd, wsums, wcodes = o.act_quantize(kind, x, 1, n)
            assert (codes == wcodes).all(), case["name"]
            assert_same(d, wd, case["name"])
            cs = codes.astype(np.int32).reshape(-1, 32).sum(axis=1)
            assert (sums == cs).all(), case["name"]
            if kind == o.ACT_Q8K:
                assert (sums == wsums).all()


def test_act_quant_nonfinite_and_zero_blocks(S):
    rs = np.random.default_rng(5)
    x = rs.standard_normal(8 * 512).astype(np.float32)
    x[3] = np.nan
    x[300] = np.inf
    x[1024:1024 + 256] = 0.0
    x[2048 + 7] = -1e-39  # subnormal maximum: the inverse scale overflows
    x[2048:2048 + 256][np.arange(256) != 7] = 0.0
    for ty, kind in ((S.WeightType.Q4_0, o.ACT_Q8_0), (S.WeightType.Q4K, o.ACT_Q8K)):
        announce(f"act_quant nonfinite {ty}")
        ws = S.new_workspace(ty, 8, 512)
        S.quantize_into(ty, dev(x), 8, 512, ws)
        codes, d, sums = read_act(ws, kind, 8, 512)
        wd, _, wcodes = o.act_quantize(kind, x, 8, 512)
        assert (codes == wcodes).all()
        assert_same(d, wd)


# ---- GEMV pinned outputs (crates/kernels-cpu/src/gemv/tests.rs:726-777) ---------------------
@pytest.mark.parametrize("ty", QTYPES)
def test_gemv_outputs_are_pinned(S, ty):
    from test_oracle_pins import PINNED
    announce(f"gemv pinned {ty}")
    rng = GemvRng(11)
    k = gemv_widths(ty)[1]
    w = gemv_weights(rng, ty, 3, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, 2, k)
    y = gpu_gemv(S, ty, w, 3, k, x, 2)
    assert bits(y).ravel().tolist() == PINNED[ty]


def test_gemv_hand_computed(S):
    announce("gemv hand computed")
    x = np.array([127.0 - i for i in range(32)], dtype=np.float32)
    one = o.f16_bits(1.0).to_bytes(2, "little")
    w = np.frombuffer(one + bytes(1 if i % 2 == 0 else 0xFF for i in range(32)), np.uint8)
    assert gpu_gemv(S, o.Q8_0, w, 1, 32, x, 1)[0, 0] == 16.0
    w = np.frombuffer(one + bytes([0x99] * 16), np.uint8)
    assert gpu_gemv(S, o.Q4_0, w, 1, 32, x, 1)[0, 0] == 3568.0
    sc = bytearray(12)
    sc[0] = 1
    sc[4] = 1
    w = np.frombuffer(one + one + bytes(sc) + bytes([0x22] * 128), np.uint8)
    xk = np.zeros(256, np.float32)
    xk[:32] = 127.0
    assert gpu_gemv(S, o.Q4_K, w, 1, 256, xk, 1)[0, 0] == 32.0 * 127.0


@pytest.mark.parametrize("ty", QTYPES)
def test_gemv_equals_oracle_random_shapes(S, ty):
    """gemv/tests.rs:284-301 shapes: every width, rows 1..16, on the GPU against the oracle."""
    rng = GemvRng(1)
    for k in gemv_widths(ty):
        for rows in (1, 2, 3, 5, 8, 9, 16):
            n_out = 7
            announce(f"gemv random ty={ty} k={k} rows={rows}")
            w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
            x = gemv_activations(rng, rows, k)
            assert_same(gpu_gemv(S, ty, w, n_out, k, x, rows), o.gemv(ty, w, n_out, k, x, rows),
                        f"ty {ty} k {k} rows {rows}")


@pytest.mark.parametrize("ty", QTYPES)
def test_gemv_unaligned_weights(S, ty):
    """gemv/tests.rs:799-817: weights at an odd address give the same bits."""
    rng = GemvRng(13)
    k = gemv_widths(ty)[2]
    n_out = 9
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    for rows in (1, 3):
        x = gemv_activations(rng, rows, k)
        want = o.gemv(ty, w, n_out, k, x, rows)
        xd = dev(x)
        for shift in (1, 2, 3, 16):
            announce(f"gemv unaligned ty={ty} rows={rows} shift={shift}")
            buf = torch.zeros(w.size + 32, dtype=torch.uint8, device="cuda")
            buf[shift:shift + w.size] = dev(w)
            W = S.Weights(ty, buf[shift:shift + w.size], n_out, k)
            assert_same(host(S.gemv(W, xd, rows)), want, f"rows {rows} shift {shift}")


def test_gemv_edge_cases(S):
    """gemv/tests.rs:460-547, 780-795: NaN/inf rows, NaN scales, zero activations, zero width."""
    rng = GemvRng(4)
    for ty in QTYPES:
        k = gemv_widths(ty)[0]
        n_out = 4
        announce(f"gemv edges ty={ty}")
        w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
        x = gemv_activations(rng, 2, k)
        x[k + k // 2] = np.nan
        y = gpu_gemv(S, ty, w, n_out, k, x, 2)
        assert not np.isnan(y[0]).any() and np.isnan(y[1]).all()
        x[k + k // 2] = np.inf
        y = gpu_gemv(S, ty, w, n_out, k, x, 2)
        assert np.isnan(y[1]).all()
        w2 = w.copy()
        rb = o.row_bytes(ty, k)
        w2[rb:rb + 2] = np.frombuffer((0x7E00).to_bytes(2, "little"), np.uint8)
        y = gpu_gemv(S, ty, w2, n_out, k, gemv_activations(rng, 1, k), 1)
        assert np.isnan(y[0, 1]) and not np.isnan(y[0, [0, 2, 3]]).any()
        y = gpu_gemv(S, ty, w, n_out, k, np.zeros(3 * k, np.float32), 3)
        assert (bits(y) == 0).all()
        y = gpu_gemv(S, ty, w, n_out, k, np.full(2 * k, 3.0e38, np.float32), 2)
        assert_same(y, o.gemv(ty, w, n_out, k, np.full(2 * k, 3.0e38, np.float32), 2))
        # zero width: every output +0
        W0 = S.Weights(ty, torch.zeros(0, dtype=torch.uint8, device="cuda"), 3, 0)
        y0 = torch.full((2, 3), 7.0, device="cuda")
        S.gemv(W0, torch.zeros(16, device="cuda"), 2, y=y0)
        assert (bits(host(y0)) == 0).all()


def test_gemv_refusals(S):
    with pytest.raises(S.GemvError):
        S.Weights(S.WeightType.Q4_0, torch.zeros(18, dtype=torch.uint8, device="cuda"), 1, 16)
    with pytest.raises(S.GemvError):
        S.Weights(S.WeightType.Q8_0, torch.zeros(33, dtype=torch.uint8, device="cuda"), 1, 32)
    W = S.Weights(S.WeightType.Q8_0, torch.zeros(34, dtype=torch.uint8, device="cuda"), 1, 32)
    with pytest.raises(S.GemvError):
        S.gemv(W, torch.zeros(31, device="cuda"), 1)
    ws = torch.zeros(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(S.SynError) as e:
        S.gemv(W, torch.zeros(32, device="cuda"), 1, ws=ws)
    assert e.value.code == 3


# ---- config shapes ----------------------------------------------------------------------------
def normal_weights(ty, n_out, k, seed):
    x = o.normal(seed, 0.02, n_out * k)
    return o.quantize(ty, x)


CONFIG_SHAPES = [
    ("cfg1 Q4_0 4096x4096", o.Q4_0, 4096, 4096, [1]),
    ("cfg2 Q8_0 14336x4096", o.Q8_0, 14336, 4096, [1, 8, 32, 128]),
    ("cfg3 QKV", o.Q4_K, 6144, 4096, [1]),
    ("cfg3 O", o.Q4_K, 4096, 4096, [1]),
    ("cfg3 gate", o.Q4_K, 14336, 4096, [1]),
    ("cfg3 down", o.Q4_K, 4096, 14336, [1]),
]


@pytest.mark.parametrize("name,ty,n_out,k,rowss", CONFIG_SHAPES, ids=[c[0] for c in CONFIG_SHAPES])
def test_gemv_config_shapes_bit_exact(S, name, ty, n_out, k, rowss):
    w = normal_weights(ty, n_out, k, 0x51A10000 + n_out + k)
    wd = dev(w)
    for rows in rowss:
        announce(f"gemv config {name} rows={rows}")
        x = o.normal(0x51A20000 + rows, 1.0, rows * k)
        want = o.gemv(ty, w, n_out, k, x, rows, threads=8)
        got = host(S.gemv(S.Weights(ty, wd, n_out, k), dev(x), rows))
        assert_same(got, want, f"{name} rows {rows}")


@pytest.mark.parametrize("k", [256, 1536, 4096, 14336])
def test_gemv_q4k_decode_paths_agree(S, k):
    """The one-launch Q4_K decode path (activation row quantized in LDS) and the two-launch
    path (quantize into the workspace, then GEMV) equal the oracle, for every K of the configs."""
    n_out = 300
    w = normal_weights(o.Q4_K, n_out, k, 0x51A30000 + k)
    x = o.normal(0x51A40000 + k, 1.0, k)
    want = o.gemv(o.Q4_K, w, n_out, k, x, 1)
    W = S.Weights(S.WeightType.Q4K, dev(w), n_out, k)
    announce(f"q4k decode fused k={k}")
    assert_same(host(S.gemv(W, dev(x), 1)), want, "fused")
    ws = S.new_workspace(S.WeightType.Q4K, 1, k)
    S.quantize_into(S.WeightType.Q4K, dev(x), 1, k, ws)
    y = torch.empty(n_out, device="cuda")
    announce(f"q4k decode ws k={k}")
    S.gemv_quantized(W, ws, 1, y)
    assert_same(host(y), want, "workspace")


def test_gemv_batch_layer_shapes(S):
    """The grouped decode launch equals the oracle on every problem of a Q4_K decode layer
    (Llama-3-8B shapes, output rows cut to keep the oracle quick) plus odd shapes."""
    shapes = [(6144, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336),
              (37, 256), (5, 1536), (1, 16384)]
    # every row width the kernel picks: 16 lanes (K <= 4096), 32 (<= 8192), 64 (<= 16384)
    Ws, xs, ys, want = [], [], [], []
    for i, (n_out, k) in enumerate(shapes):
        n = min(n_out, 1024)
        w = normal_weights(o.Q4_K, n, k, 0x51A50000 + i)
        x = o.normal(0x51A60000 + i, 1.0, k)
        want.append(o.gemv(o.Q4_K, w, n, k, x, 1))
        Ws.append(S.Weights(S.WeightType.Q4K, dev(w), n, k))
        xs.append(dev(x))
        ys.append(torch.full((n,), float("nan"), device="cuda"))
    announce("gemv batch layer")
    batch = S.GemvBatch(Ws, xs, ys)
    for rep in range(3):
        batch()
        for i in range(len(shapes)):
            assert_same(host(ys[i]), want[i], f"problem {i} rep {rep}")
    # the two halves (quantize, then the GEMV on the Q8_K rows) give the same bits
    for y in ys:
        y.fill_(float("nan"))
    batch.quantize()
    batch.gemv_quantized()
    for i in range(len(shapes)):
        assert_same(host(ys[i]), want[i], f"problem {i} split")


def test_gemv_batch_row_widths(S):
    """K of 17..32 and 33..64 super-blocks (32- and 64-lane rows) and ragged row counts."""
    shapes = [(50, 5120), (3, 8192), (65, 8448), (9, 12288), (130, 2048)]
    Ws, xs, ys, want = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        w = normal_weights(o.Q4_K, n, k, 0x51A70000 + i)
        x = o.normal(0x51A80000 + i, 1.0, k)
        want.append(o.gemv(o.Q4_K, w, n, k, x, 1))
        Ws.append(S.Weights(S.WeightType.Q4K, dev(w), n, k))
        xs.append(dev(x))
        ys.append(torch.full((n,), float("nan"), device="cuda"))
    announce("gemv batch row widths")
    S.GemvBatch(Ws, xs, ys)()
    for i in range(len(shapes)):
        assert_same(host(ys[i]), want[i], f"problem {i}")


# ---- weight packing and dequant ----------------------------------------------------------
@pytest.mark.parametrize("ty", QTYPES)
def test_quantize_equals_ggml_bytes(S, ty):
    from test_oracle_pins import DIGESTS, SEEDS
    for seed, want in zip(SEEDS, DIGESTS[ty]):
        announce(f"quantize digest ty={ty} seed={seed:#x}")
        q = host(S.quantize(ty, dev(quant_values(seed, 256 * 64))))
        assert o.fnv1a(q) == want
    x = o.normal(77, 0.02, 256 * 4096)
    announce(f"quantize normal ty={ty}")
    assert (host(S.quantize(ty, dev(x))) == o.quantize(ty, x)).all()


@pytest.mark.parametrize("ty", QTYPES)
def test_dequantize_exact(S, ty):
    rng = GemvRng(21)
    w = gemv_weights(rng, ty, 16, 512, o.f16_bits, o.round_bf16)
    announce(f"dequantize ty={ty}")
    assert_same(host(S.dequantize(ty, dev(w))), o.dequantize(ty, w))


def test_every_f16_scale_converts_exactly(S):
    """The device F16->F32 conversion on every pattern, through Q8_0 dequant with code 1."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0] = h & 0xFF
    blocks[:, 1] = h >> 8
    blocks[:, 2:] = 1
    announce("f16 patterns")
    got = host(S.dequantize(o.Q8_0, dev(blocks.ravel()))).reshape(65536, 32)[:, 0]
    assert_same(got, o.dequantize(o.Q8_0, blocks.ravel()).reshape(65536, 32)[:, 0])


# ---- GateUpAct{Silu}: the Gemv of the stacked [gate; up] weight, then silu(g) * u --------------
@pytest.mark.parametrize("ty,rows,n,k", [(o.Q4_K, 1, 1536, 4096), (o.Q4_K, 5, 700, 2048),
                                         (o.Q4_K, 96, 512, 4096), (o.Q8_0, 1, 1000, 4096),
                                         (o.Q4_0, 9, 333, 1024)])
def test_gate_up_act_equals_oracle(S, ty, rows, n, k):
    rng = GemvRng(ty * 17 + rows * 3 + n)
    w = gemv_weights(rng, ty, 2 * n, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    announce(f"gate_up_act ty={ty} rows={rows} n={n} k={k}")
    W = S.Weights(ty, dev(w), 2 * n, k)
    got = host(S.gate_up_act(W, dev(x.astype(np.float32)), rows))
    assert_same(got, o.gate_up_act(ty, w, n, k, x, rows, threads=8), "gate_up_act")


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
@pytest.mark.parametrize("n,k", [(700, 4096), (64, 45056)])
def test_gate_up_act_split_layout(S, ty, n, k):
    """GateUpAct over SPLIT weights: one row (one launch that quantizes the row in LDS at 4096
    values; the quantization launch first at 45,056), a few rows and the GEMM's row counts."""
    rng = GemvRng(ty * 31 + n + k)
    w = gemv_weights(rng, ty, 2 * n, k, o.f16_bits, o.round_bf16)
    W = S.repack(S.Weights(ty, dev(w), 2 * n, k))
    assert W.layout == S.LAYOUT_SPLIT
    for rows in (1, 3, 12):
        x = gemv_activations(rng, rows, k)
        announce(f"gate_up_act split ty={ty} rows={rows} n={n} k={k}")
        got = host(S.gate_up_act(W, dev(x.astype(np.float32)), rows))
        assert_same(got, o.gate_up_act(ty, w, n, k, x, rows, threads=8), f"split rows {rows}")


def test_gate_up_act_x8_layout(S):
    rng = GemvRng(4242)
    n, k = 1024, 4096
    w = gemv_weights(rng, o.Q4_K, 2 * n, k, o.f16_bits, o.round_bf16)
    for rows in (1, 64):
        x = gemv_activations(rng, rows, k)
        announce(f"gate_up_act x8 rows={rows}")
        W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), 2 * n, k))
        got = host(S.gate_up_act(W, dev(x.astype(np.float32)), rows))
        assert_same(got, o.gate_up_act(o.Q4_K, w, n, k, x, rows, threads=8), f"x8 rows {rows}")


@pytest.mark.parametrize("n,k", [(14336, 4096), (37, 4096), (500, 14336), (129, 8192), (3, 256)])
def test_gate_up_act_x8_one_row_fused(S, n, k):
    """One row over X8 weights runs gate, up and silu(g) u in one launch (the gate and up rows of
    an output side by side): the Llama-3-8B FFN shape, ragged row counts, and 16-, 32- and
    64-lane rows."""
    from test_gpu_gemm import random_q4k
    rs = np.random.default_rng(n + k)
    w = random_q4k(rs, 2 * n, k)
    x = o.normal(0x6A7E + n, 1.0, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), 2 * n, k))
    announce(f"gate_up_act x8 fused n={n} k={k}")
    got = host(S.gate_up_act(W, dev(x), 1))
    assert_same(got, o.gate_up_act(o.Q4_K, w, n, k, x, 1, threads=16), "fused gate_up_act")


# ---- F16 / BF16 weights: 32 FMA accumulators and the halving fold (portable.rs:30-45) ----------
@pytest.mark.parametrize("ty", [o.F16, o.BF16])
@pytest.mark.parametrize("rows,n_out,k", [(1, 4096, 4096), (3, 1000, 1024), (9, 64, 4096),
                                          (7, 513, 40), (2, 100, 33), (1, 5, 7)])
def test_float_gemv_equals_oracle(S, ty, rows, n_out, k):
    """Rows of 8-element-aligned k take 16-byte loads, others one element at a time; more than
    four activation rows run in groups of four over the same weight chunks."""
    rng = GemvRng(ty * 31 + rows * 7 + k)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    announce(f"float gemv ty={ty} rows={rows} n_out={n_out} k={k}")
    got = gpu_gemv(S, ty, w, n_out, k, x, rows)
    assert_same(got, o.gemv(ty, w, n_out, k, x, rows, threads=8), f"ty {ty}")


def test_float_gemv_golden_case(S):
    """The pinned output bits of crates/kernels-cpu/src/gemv/tests.rs:726-777 on the device."""
    from test_oracle_pins import PINNED
    for ty in (o.F16, o.BF16):
        rng = GemvRng(11)
        k = gemv_widths(ty)[1]
        w = gemv_weights(rng, ty, 3, k, o.f16_bits, o.round_bf16)
        x = gemv_activations(rng, 2, k)
        announce(f"float gemv golden ty={ty}")
        got = gpu_gemv(S, ty, w, 3, k, x, 2)
        assert bits(got).ravel().tolist() == PINNED[ty]
