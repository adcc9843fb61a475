"""Pins of the CPU oracle against what the reference itself records.

Each test cites the reference test or data it reproduces.  These run on the CPU only.
"""
import os

import numpy as np
import pytest

from oracle import oracle as o
from refgen import (GemvRng, MoeRng, gemv_activations, gemv_weights, gemv_widths, moe_activations,
                    moe_matrix, moe_route_ids, quant_values)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TYPES = [o.F16, o.BF16, o.Q8_0, o.Q4_0, o.Q4_K]


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- crates/kernels-cpu/src/gemv/tests.rs:726-777 outputs_are_pinned -----------------------
PINNED = {
    o.F16: [0x420A1B10, 0x454B51BA, 0xC3D1653B, 0x3FC76C70, 0xC028A29A, 0x3F9AB456],
    o.BF16: [0x420A439A, 0x454BA9FA, 0xC3D0EE64, 0x3FC733F4, 0xC02A34AE, 0x3F9A739A],
    o.Q8_0: [0x40A0ABE7, 0xC2AB4CC2, 0x41FC936A, 0x4094D860, 0xC1B6724A, 0xC089CC5F],
    o.Q4_0: [0xBE40FE75, 0xBF1A503E, 0x408F99D8, 0x3F152B45, 0xBFBC2046, 0x3F151262],
    o.Q4_K: [0x43065438, 0xC5CB1506, 0x4353F838, 0x43517B96, 0xC596E5A0, 0x44910FBE],
}


def golden_case(ty):
    rng = GemvRng(11)
    k = gemv_widths(ty)[1]
    w = gemv_weights(rng, ty, 3, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, 2, k)
    return o.gemv(ty, w, 3, k, x, 2)


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_outputs_are_pinned(ty):
    got = bits(golden_case(ty)).ravel().tolist()
    assert got == PINNED[ty], [hex(v) for v in got]


# ---- gemv/tests.rs:407-458 hand_computed_cases ----------------------------------------
def test_gemv_hand_computed_cases():
    x = np.array([127.0 - i for i in range(32)], dtype=np.float32)
    one = o.f16_bits(1.0).to_bytes(2, "little")
    w = np.frombuffer(one + bytes(1 if i % 2 == 0 else 0xFF for i in range(32)), np.uint8)
    assert o.gemv(o.Q8_0, w, 1, 32, x, 1)[0, 0] == 16.0
    w = np.frombuffer(one + bytes([0x99] * 16), np.uint8)
    assert o.gemv(o.Q4_0, w, 1, 32, x, 1)[0, 0] == 3568.0
    x33 = np.arange(1, 34, dtype=np.float32)
    w = np.frombuffer(b"".join(o.f16_bits(2.0).to_bytes(2, "little") for _ in range(33)), np.uint8)
    assert o.gemv(o.F16, w, 1, 33, x33, 1)[0, 0] == 1122.0
    w = np.frombuffer(b"".join(o.round_bf16(2.0).to_bytes(2, "little") for _ in range(33)), np.uint8)
    assert o.gemv(o.BF16, w, 1, 33, x33, 1)[0, 0] == 1122.0
    scales = bytearray(12)
    scales[0] = 1
    scales[4] = 1
    w = np.frombuffer(one + one + bytes(scales) + bytes([0x22] * 128), np.uint8)
    xk = np.zeros(256, np.float32)
    xk[:32] = 127.0
    assert o.gemv(o.Q4_K, w, 1, 256, xk, 1)[0, 0] == 32.0 * 127.0


def test_gate_up_act_one_hot_rows():
    """GateUpAct{Silu} (linear.rs:75-112) on the stacked [gate; up] weight of the ggml binding
    (kernels-ggml/src/mapping.rs:31): with one-hot Q8_0 rows each dot is one activation code
    times its scale, so the output pins the row order (gate rows first) and silu(g) * u."""
    one = o.f16_bits(1.0).to_bytes(2, "little")

    def row(j):
        return np.frombuffer(one + bytes(1 if i == j else 0 for i in range(32)), np.uint8)

    x = np.linspace(-3.0, 2.5, 32).astype(np.float32)
    picks = (3, 7, 20, 31)  # gate rows 0, 1; up rows 0, 1
    w = np.concatenate([row(j) for j in picks])
    y = o.gate_up_act(o.Q8_0, w, 2, 32, x, 1)[0]
    dot = [np.float32(o.gemv(o.Q8_0, row(j), 1, 32, x, 1)[0, 0]) for j in picks]
    want = [np.float32(o.silu(float(dot[i]))) * dot[2 + i] for i in range(2)]
    assert bits(y).tolist() == bits(np.array(want, np.float32)).tolist()
    swapped = [np.float32(o.silu(float(dot[2 + i]))) * dot[i] for i in range(2)]
    assert bits(y).tolist() != bits(np.array(swapped, np.float32)).tolist()


def test_gemv_zero_activations_give_positive_zero():
    """gemv/tests.rs:780-795."""
    rng = GemvRng(12)
    for ty in TYPES:
        k = gemv_widths(ty)[1]
        w = gemv_weights(rng, ty, 5, k, o.f16_bits, o.round_bf16)
        y = o.gemv(ty, w, 5, k, np.zeros(3 * k, np.float32), 3)
        assert (bits(y) == 0).all(), ty


def exact_parts(ty, w, k):
    """gemv/tests.rs:184-214: the weights in F64 as two parts (Q4_K: d*sc*q and -dmin*m)."""
    if ty != o.Q4_K:
        return o.dequantize(ty, w).astype(np.float64), np.zeros(w.size // o.BLOCK_BYTES[ty] * o.BLOCK_ELEMS[ty])
    a, b = [], []
    for blk in w.reshape(-1, 144):
        d = float(o.f16_to_f32(int(blk[0]) | int(blk[1]) << 8))
        dmin = float(o.f16_to_f32(int(blk[2]) | int(blk[3]) << 8))
        sc = blk[4:16]
        q = blk[16:]
        for g in range(4):
            for hi in (0, 1):
                j = 2 * g + hi
                if j < 4:
                    s, m = sc[j] & 63, sc[j + 4] & 63
                else:
                    s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
                    m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
                for l in range(32):
                    n = (q[32 * g + l] >> 4) if hi else (q[32 * g + l] & 0xF)
                    a.append(d * s * n)
                    b.append(-dmin * m)
    return np.array(a), np.array(b)


def seen(ty, x, rows, k):
    """The activations as quantized (gemv/tests.rs:164-182)."""
    kind = o.ACT_KIND[ty]
    if kind == o.ACT_F32:
        return x.astype(np.float64).reshape(rows, k)
    d, _, codes = o.act_quantize(kind, x, rows, k)
    blk = 32 if kind == o.ACT_Q8_0 else 256
    return (codes.astype(np.float32).reshape(-1, blk) * d[:, None]).astype(np.float64).reshape(rows, k)


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_within_the_derived_bound(ty):
    """gemv/tests.rs:217-272: |y - exact| <= n * 2^-24 * sum|w x| against F64."""
    rng = GemvRng(2)
    U = 2.0**-24
    for k in gemv_widths(ty)[:3]:
        for rows in (1, 4):
            n_out = 5
            w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
            x = gemv_activations(rng, rows, k)
            y = o.gemv(ty, w, n_out, k, x, rows).astype(np.float64)
            a, b = exact_parts(ty, w, k)
            a, b = a.reshape(n_out, k), b.reshape(n_out, k)
            xs = seen(ty, x, rows, k)
            exact = xs @ (a + b).T
            mag = np.abs(xs) @ (np.abs(a) + np.abs(b)).T
            kn = (k // 32 + 1 + 5) if ty in (o.F16, o.BF16) else (k // o.BLOCK_ELEMS[ty] + 5)
            assert (np.abs(y - exact) <= kn * U * mag + 1e-38).all(), (ty, k, rows)


def test_partition_covers_every_row_once():
    """gemv/tests.rs:549-580."""
    for ty in TYPES:
        for k in gemv_widths(ty)[:2]:
            for n_out in (0, 1, 7, 64, 100, 4097):
                for parts in (0, 1, 2, 3, 8, 13, 200):
                    runs = o.partition(ty, n_out, k, parts)
                    assert len(runs) == max(parts, 1)
                    nxt = 0
                    for s, e in runs:
                        assert s == min(nxt, n_out) and s <= e
                        nxt = e
                    assert nxt == n_out


def test_threaded_gemv_equals_one_thread():
    rng = GemvRng(5)
    for ty in TYPES:
        k = gemv_widths(ty)[1]
        w = gemv_weights(rng, ty, 37, k, o.f16_bits, o.round_bf16)
        x = gemv_activations(rng, 3, k)
        want = o.gemv(ty, w, 37, k, x, 3)
        for t in (2, 3, 5, 16):
            assert (bits(o.gemv(ty, w, 37, k, x, 3, threads=t)) == bits(want)).all()


# ---- crates/kernels-ggml/tests/quantize.rs:114-161 digests ---------------------------------
DIGESTS = {
    o.Q4_K: (0x6618701AAA7359E9, 0x9E84FC732A4F55DE),
    o.Q8_0: (0x4C103906FF52CFAC, 0x259BCEF0EA1BCF85),
    o.Q4_0: (0x7E8110B4C98A9DE1, 0x61E62FE744AD866A),
    o.BF16: (0xA4ACEAF11D9B1E15, 0x1E32D4A9CBDDBCA1),
    o.F16: (0x7B60211630C50897, 0x8B8F62832A16DC77),
}
SEEDS = (1, 0x5EEDF1C57E570007)


@pytest.fixture(scope="module")
def quant_inputs():
    return {s: quant_values(s, 256 * 64) for s in SEEDS}


@pytest.mark.parametrize("ty", [o.Q4_K, o.Q8_0, o.Q4_0, o.BF16, o.F16])
def test_quantizer_digests(ty, quant_inputs):
    for seed, want in zip(SEEDS, DIGESTS[ty]):
        q = o.quantize(ty, quant_inputs[seed])
        assert q.size == 256 * 64 // o.BLOCK_ELEMS[ty] * o.BLOCK_BYTES[ty]
        assert o.fnv1a(q) == want, (ty, hex(seed), hex(o.fnv1a(q)))


def test_quantizers_equal_ggml_own_build(quant_inputs):
    """Where oracle/_ref was built from the reference's ggml-quants.c, byte-compare."""
    R = o.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent here)")
    rs = np.random.default_rng(7)
    cases = [quant_inputs[SEEDS[0]], (rs.standard_normal(256 * 32) * 0.02).astype(np.float32)]
    for x in cases:
        for ty in (o.Q4_0, o.Q8_0, o.Q4_K):
            want = np.zeros(o.row_bytes(ty, x.size), np.uint8)
            R.ref_quantize(ty, x.ctypes.data, x.size, want.ctypes.data)
            got = o.quantize(ty, x)
            assert (got == want).all(), ty
            back = np.zeros(x.size, np.float32)
            R.ref_dequantize(ty, got.ctypes.data, x.size, back.ctypes.data)
            assert (bits(o.dequantize(ty, got)) == bits(back)).all(), ty


# ---- crates/kernels/tests/data/act_quant/ggml-q8.txt ---------------------------------------
def load_act_cases():
    cases = []
    cur = None
    with open(os.path.join(GOLDEN, "act_quant", "ggml-q8.txt")) as f:
        for line in f:
            line = line.strip()
            if line.startswith("case "):
                _, name, n = line.split()
                cur = {"name": name, "n": int(n)}
            elif line.startswith("in ") and cur is not None:
                h = line[3:]
                cur["in"] = np.array([int(h[i:i + 8], 16) for i in range(0, len(h), 8)],
                                     dtype=np.uint32).view(np.float32)
            elif line == "end":
                cases.append(cur)
                cur = None
            elif cur is not None and line:
                parts = line.split()
                cur[parts[0] + " " + parts[1]] = bytes.fromhex(parts[2])
    return cases


ACT_CASES = load_act_cases()


def test_act_vectors_loaded():
    assert len(ACT_CASES) == 20
    assert all("in" in c for c in ACT_CASES)


@pytest.mark.parametrize("case", ACT_CASES, ids=[c["name"] for c in ACT_CASES])
def test_act_quant_golden(case):
    x = case["in"]
    n = x.size
    if "q8_0 ref" in case:
        assert o.q8_0_blocks(x, 0).tobytes() == case["q8_0 ref"]
        assert o.q8_0_blocks(x, 1).tobytes() == case["q8_0 cpu"]
        assert o.q8_1_blocks(x, 0).tobytes() == case["q8_1 ref"]
        assert o.q8_1_blocks(x, 1).tobytes() == case["q8_1 cpu"]
        # the GEMV workspace quantizer (gemv/act.rs) equals the arm64 path's codes and F16 scale
        d, _, codes = o.act_quantize(o.ACT_Q8_0, x, 1, n)
        want = np.frombuffer(case["q8_0 cpu"], np.uint8).reshape(-1, 34)
        assert (codes.view(np.uint8).reshape(-1, 32) == want[:, 2:]).all()
        dh = want[:, 0].astype(np.uint16) | (want[:, 1].astype(np.uint16) << 8)
        assert (bits(d) == bits([o.f16_to_f32(int(h)) for h in dh])).all()
    if "q8_K ref" in case:
        assert o.q8_k_blocks(x).tobytes() == case["q8_K ref"]
        assert case["q8_K cpu"] == case["q8_K ref"]
        d, sums, codes = o.act_quantize(o.ACT_Q8K, x, 1, n)
        want = np.frombuffer(case["q8_K ref"], np.uint8).reshape(-1, 292)
        assert (bits(d) == want[:, :4].copy().view(np.uint32).ravel()).all()
        assert (codes.view(np.uint8).reshape(-1, 256) == want[:, 4:260]).all()
        bs = want[:, 260:].copy().view(np.int16).reshape(-1, 8, 2).sum(axis=2)
        assert (sums.reshape(-1, 8) == bs).all()
    if "f16 ref" in case:
        want = np.frombuffer(case["f16 ref"], np.uint16)
        assert [o.f16_bits(float(v)) for v in x] == want.tolist()
    if "bf16 ref" in case:
        want = np.frombuffer(case["bf16 ref"], np.uint16)
        assert [o.round_bf16(float(v)) for v in x] == want.tolist()


# ---- conversions and math ----------------------------------------------------------------
def test_f16_to_f32_every_pattern():
    for h in range(0, 1 << 16, 1):
        v = np.float32(o.f16_to_f32(h))
        ref = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        if np.isnan(ref):
            assert np.isnan(v)
        else:
            assert bits(v) == bits(ref), hex(h)


def test_f16_bits_matches_ieee_rne():
    rs = np.random.default_rng(3)
    xs = np.concatenate([
        rs.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rs.integers(-30, 17, 20000).astype(np.float32),
        np.array([65504, 65519.99, 65520, 6e-8, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0], np.float32),
    ]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([o.f16_bits(float(v)) for v in xs], np.uint16)
    assert (got == want).all()


def test_exp_within_two_ulp():
    """crates/kernels/src/reference/math/tests.rs:19-40 (every 97th bit pattern)."""
    assert o.exp_worst_ulp(97) <= 2.0


def test_exp_and_silu_edge_cases():
    """math/tests.rs:42-84."""
    assert o.exp(0.0) == 1.0 and o.exp(-0.0) == 1.0
    assert o.exp(float("inf")) == float("inf")
    assert bits(o.exp(float("-inf"))) == 0
    assert o.exp(88.72284) == float("inf") and o.exp(100.0) == float("inf")
    assert bits(o.exp(-104.0)) == 0
    tiny = o.exp(-100.0)
    assert 0 < tiny < np.finfo(np.float32).tiny
    assert bits(o.silu(0.0)) == 0 and bits(o.silu(-0.0)) == 0x80000000
    assert o.silu(float("inf")) == float("inf")
    assert np.isnan(o.silu(float("-inf")))
    assert bits(o.silu(-100.0)) == 0x80000000
    assert o.silu(20.0) == 20.0


def level_by_level(ts):
    """reduce.rs module docs written out: blocks of 32 summed in order, then pairwise."""
    ts = [np.float32(t) for t in ts]
    if not ts:
        return np.float32(0.0)
    sums = []
    for s in range(0, len(ts), 32):
        acc = np.float32(0.0)
        for t in ts[s:s + 32]:
            acc = np.float32(acc + t)
        sums.append(acc)
    while len(sums) > 1:
        nxt = [np.float32(sums[i] + sums[i + 1]) for i in range(0, len(sums) - 1, 2)]
        if len(sums) % 2:
            nxt.append(sums[-1])
        sums = nxt
    return sums[0]


def test_f32fixed_sum_equals_the_level_by_level_tree():
    rs = np.random.default_rng(11)
    for n in [0, 1, 31, 32, 33, 64, 65, 95, 96, 97, 128, 160, 1000, 4096, 4097]:
        xs = (rs.standard_normal(n) * 10.0 ** rs.integers(-3, 4, n)).astype(np.float32)
        assert bits(o.fsum(xs)) == bits(level_by_level(xs)), n
        b = rs.standard_normal(n).astype(np.float32)
        assert bits(o.fdot(xs, b)) == bits(level_by_level(xs * b)), n


# ---- crates/kernels-cpu/src/moe/tests.rs: the grouped expert FFN --------------------------------
MOE = (6, 2, 256, 512)  # n_experts, top_k, hidden, inter (moe/tests.rs:227-236)
SENTINEL = 0x7FC0DEAD


def moe_layer(seed):
    e, _, hidden, inter = MOE
    rng = MoeRng(seed)
    gate = moe_matrix(rng, o.Q4_K, e * inter, hidden, o.f16_bits)
    up = moe_matrix(rng, o.Q4_K, e * inter, hidden, o.f16_bits)
    down = moe_matrix(rng, o.Q4_K, e * hidden, inter, o.f16_bits)
    return rng, gate, up, down


def ffn_alone(gate, up, down, e, x):
    """moe/tests.rs:300-313: one row through expert e's gate/up Gemv, silu(g) * u, down Gemv,
    from the pinned Gemv and activation quantizer."""
    _, _, hidden, inter = MOE
    gb, db = inter * o.row_bytes(o.Q4_K, hidden), hidden * o.row_bytes(o.Q4_K, inter)
    g = o.gemv(o.Q4_K, gate[e * gb:(e + 1) * gb], inter, hidden, x, 1)[0]
    u = o.gemv(o.Q4_K, up[e * gb:(e + 1) * gb], inter, hidden, x, 1)[0]
    h = np.array([np.float32(o.silu(float(a))) * b for a, b in zip(g, u)], np.float32)
    return o.gemv(o.Q4_K, down[e * db:(e + 1) * db], hidden, inter, h, 1)[0]


def test_moe_every_slot_is_its_experts_ffn_of_the_row_alone():
    """moe/tests.rs:315-337."""
    rng, gate, up, down = moe_layer(1)
    n_experts, top_k, hidden, inter = MOE
    for rows in [1, 2, 5, 8, 9, 17]:
        x = moe_activations(rng, rows * hidden).reshape(rows, hidden)
        ids = moe_route_ids(rng, rows, top_k, n_experts)
        out = o.moe_grouped(o.Q4_K, o.Q4_K, n_experts, top_k, hidden, inter, gate, up, down, x, ids)
        for r in range(rows):
            for j in range(top_k):
                want = ffn_alone(gate, up, down, int(ids[r, j]), x[r])
                assert (bits(out[r, j]) == bits(want)).all(), (rows, r, j)


def q8_0_layer(seed):
    e, _, hidden, inter = MOE
    rng = MoeRng(seed)
    gate = moe_matrix(rng, o.Q8_0, e * inter, hidden, o.f16_bits)
    up = moe_matrix(rng, o.Q8_0, e * inter, hidden, o.f16_bits)
    down = moe_matrix(rng, o.Q8_0, e * hidden, inter, o.f16_bits)
    return rng, gate, up, down


def ffn_alone_q8_0(gate, up, down, e, x, h_q8k=False, swap=False):
    """The Q8_0-expert form of moe/tests.rs:300-313: gate/up Gemv on the row's Q8_0 blocks,
    silu(g) * u, h requantized as the down matrix's activation kind (Q8_0, act.rs:31-39), down
    Gemv.  h_q8k and swap plant mistakes: h through Q8_K first, or silu taken of the up row."""
    _, _, hidden, inter = MOE
    gb, db = inter * o.row_bytes(o.Q8_0, hidden), hidden * o.row_bytes(o.Q8_0, inter)
    g = o.gemv(o.Q8_0, gate[e * gb:(e + 1) * gb], inter, hidden, x, 1)[0]
    u = o.gemv(o.Q8_0, up[e * gb:(e + 1) * gb], inter, hidden, x, 1)[0]
    if swap:
        g, u = u, g
    h = np.array([np.float32(o.silu(float(a))) * b for a, b in zip(g, u)], np.float32)
    if h_q8k:
        d, _, codes = o.act_quantize(o.ACT_Q8K, h, 1, inter)
        h = (codes.astype(np.float32).reshape(-1, 256) * d[:, None]).astype(np.float32).ravel()
    return o.gemv(o.Q8_0, down[e * db:(e + 1) * db], hidden, inter, h, 1)[0]


def test_moe_q8_0_experts_every_slot_is_its_experts_ffn_of_the_row_alone():
    """moe/tests.rs:315-337 on Q8_0 experts (moe/entry.rs:50-55): every slot of the oracle's
    grouped FFN equals its expert's FFN of its row alone, bit for bit; the same check rejects an
    h requantized as Q8_K (the Q4_K experts' kind) and gate and up swapped."""
    rng, gate, up, down = q8_0_layer(11)
    n_experts, top_k, hidden, inter = MOE
    for rows in [1, 3, 8]:
        x = moe_activations(rng, rows * hidden).reshape(rows, hidden)
        ids = moe_route_ids(rng, rows, top_k, n_experts)
        out = o.moe_grouped(o.Q8_0, o.Q8_0, n_experts, top_k, hidden, inter, gate, up, down, x, ids)
        for r in range(rows):
            for j in range(top_k):
                e = int(ids[r, j])
                want = ffn_alone_q8_0(gate, up, down, e, x[r])
                assert (bits(out[r, j]) == bits(want)).all(), (rows, r, j)
                # planted mistakes, each caught by the same bit comparison
                assert not (bits(ffn_alone_q8_0(gate, up, down, e, x[r], h_q8k=True)) == bits(want)).all()
                assert not (bits(ffn_alone_q8_0(gate, up, down, e, x[r], swap=True)) == bits(want)).all()


def test_moe_slots_of_other_sites_keep_their_values():
    """moe/tests.rs:559-590: with the site mask on the even experts, their slots equal the
    unmasked call's and every other slot keeps its bits; the odd experts' call on the same output
    then completes it."""
    rng, gate, up, down = moe_layer(6)
    n_experts, top_k, hidden, inter = MOE
    rows = 6
    x = moe_activations(rng, rows * hidden).reshape(rows, hidden)
    ids = moe_route_ids(rng, rows, top_k, n_experts)
    args = (o.Q4_K, o.Q4_K, n_experts, top_k, hidden, inter, gate, up, down, x, ids)
    every = o.moe_grouped(*args)
    even = np.arange(n_experts, dtype=np.int32) % 2 == 0
    out = np.full(rows * top_k * hidden, SENTINEL, np.uint32).view(np.float32)
    got = o.moe_grouped(*args, site=even.astype(np.int32), out=out)
    for r in range(rows):
        for j in range(top_k):
            if ids[r, j] % 2 == 0:
                assert (bits(got[r, j]) == bits(every[r, j])).all(), (r, j)
            else:
                assert (bits(got[r, j]) == SENTINEL).all(), (r, j)
    assert (ids % 2 == 1).any() and (ids % 2 == 0).any()
    done = o.moe_grouped(*args, site=(~even).astype(np.int32), out=out)
    assert (bits(done) == bits(every)).all()


# ---- the reference's x86 level (the timed CPU baseline) ---------------------------------------
@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0, o.Q4_K])
def test_x86_level_gives_the_portable_bits(ty):
    """crates/kernels-cpu/src/gemv/x86.rs's block sums with portable.rs's 8-row groups give the
    portable kernels' bits (x86.rs module docs: the sums are exact): row counts across the group
    edges, threaded by the reference's partition, and seeded extreme codes."""
    k = 1024 if ty == o.Q4_K else 512
    for n_out, rows, threads in ((37, 1, 1), (64, 7, 3), (65, 8, 2), (33, 9, 4), (40, 17, 5)):
        rng = GemvRng(n_out * 131 + rows + ty)
        w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
        x = gemv_activations(rng, rows, k)
        want = o.gemv(ty, w, n_out, k, x, rows)
        got = o.gemv(ty, w, n_out, k, x, rows, threads=threads, level=1)
        assert (bits(got) == bits(want)).all(), (n_out, rows, threads)
    # all-extreme codes: 0x80 (-128) and 0x7F weight bytes, activations of +-127
    nb = k // o.BLOCK_ELEMS[ty]
    wb = np.frombuffer(np.random.default_rng(ty).bytes(16 * nb * o.BLOCK_BYTES[ty]), np.uint8).copy()
    blocks = wb.reshape(16 * nb, o.BLOCK_BYTES[ty])
    hdr = 4 if ty == o.Q4_K else 2
    blocks[:, :2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    if ty == o.Q4_K:
        blocks[:, 2:4] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
    blocks[:, hdr:] = np.where(blocks[:, hdr:] & 1, 0x80, 0x7F) if ty == o.Q8_0 else blocks[:, hdr:]
    x = np.where(np.random.default_rng(7).random(3 * k) < 0.5, -1.0, 1.0).astype(np.float32)
    assert (bits(o.gemv(ty, wb, 16, k, x, 3, level=1)) == bits(o.gemv(ty, wb, 16, k, x, 3))).all()


@pytest.mark.parametrize("ty", [o.Q4_K, o.Q8_0])
def test_x86_level_moe_gives_the_portable_bits(ty):
    n_experts, top_k, hidden, inter = MOE
    rng, gate, up, down = moe_layer(21) if ty == o.Q4_K else q8_0_layer(21)
    x = moe_activations(rng, 11 * hidden).reshape(11, hidden)
    ids = moe_route_ids(rng, 11, top_k, n_experts)
    args = (ty, ty, n_experts, top_k, hidden, inter, gate, up, down, x, ids)
    assert (bits(o.moe_grouped(*args, threads=3, level=1)) == bits(o.moe_grouped(*args))).all()
