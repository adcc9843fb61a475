"""The activation quantizers in every form the kernels use them, on rows built to separate the
rules: largest magnitude with the first index on ties between +m and -m (either sign first, in
one lane or across lanes of the block), all-zero and all -0.0 blocks, subnormal maxima, and NaN
or infinity in a block (crates/kernels-cpu/src/gemv/act.rs:323-373).  Forms: the separate
Q8_K / Q8_0 quantizer, the lone Q4_K GEMV over X8 weights that quantizes its row in every
workgroup (16, 32 and 56 super-blocks: 8 and 16 wavefronts), the fused GateUpAct, the two-row
fused decode, the one-row SPLIT GEMV (Q8_0 blocks in the workgroup), and the MoE gather; each
against the oracle, bit for bit."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_gemm import random_q4k
from test_gpu_gemv import read_act

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def S():
    require_gpu()
    import syntropy_amd.gemv as S
    return S


def crafted_row(k, seed, nonfinite=None):
    """Random N(0,1) 256-value blocks, the first few replaced by tie and zero cases."""
    rs = np.random.default_rng(seed)
    x = rs.standard_normal(k).astype(np.float32)
    nb = k // 256
    cases = []
    # +m and -m in different lanes (lanes hold 16 values in the in-workgroup form, 4 in the
    # wavefront form): the first index decides the sign
    cases.append({5: -3.0, 100: 3.0})
    cases.append({7: 2.5, 200: -2.5})
    # the tie inside one lane's values, negative first and positive first
    cases.append({16: -4.0, 17: 4.0})
    cases.append({33: 4.0, 34: -4.0})
    # three equal magnitudes, the last lane's first
    cases.append({255: -1.5, 254: 1.5, 0: 1.5})
    for c, vals in enumerate(cases[:max(0, nb - 4)]):
        blk = x[c * 256:(c + 1) * 256]
        blk *= np.float32(0.25)
        for i, v in vals.items():
            blk[i] = np.float32(v)
    if nb > 6:
        x[5 * 256:6 * 256] = 0.0                      # all +0
        x[6 * 256:7 * 256] = np.float32(-0.0)         # all -0
    if nb > 8:
        x[7 * 256:8 * 256] = 0.0
        x[7 * 256 + 9] = np.float32(-1e-39)           # subnormal maximum: the inverse scale overflows
        x[8 * 256:9 * 256] *= np.float32(1e-40)       # every value subnormal
    if nb > 10:
        # the quantizers' short division forms hand over to the division at their range ends:
        # a block of normal values whose Q8_0 scale is subnormal and whose Q8_K inverse scale
        # overflows, and one whose maximum passes 2^126
        x[9 * 256:10 * 256] *= np.float32(1e-37)
        x[10 * 256:11 * 256] *= np.float32(3e37)
    if nonfinite is not None:
        x[nb // 2 * 256 + 77] = np.float32(nonfinite)
    return x


ROWS = [(4096, 11), (8192, 12), (14336, 13), (2048, 14)]


def test_division_forms_equal_the_division_everywhere(S):
    """The quantizers' short forms of amax / 127, 1 / b, -127 / b, the F16 rounding of the
    scale and the rounding of scaled values to codes equal the correctly rounded division, the
    integer F16 conversion and ggml's nearest_int for every F32 bit pattern but the NaNs (one
    launch over all 2^32)."""
    counts = torch.zeros(5, dtype=torch.int64, device="cuda")
    announce("division forms over every F32 pattern")
    assert S.lib().syn_div_forms_check(counts.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert counts.tolist() == [0, 0, 0, 0, 0]


@pytest.mark.parametrize("k,seed", ROWS)
def test_separate_quantizers(S, k, seed):
    x = np.stack([crafted_row(k, seed), crafted_row(k, seed + 1, np.nan), crafted_row(k, seed + 2, np.inf)])
    for ty, kind in ((S.WeightType.Q4_0, o.ACT_Q8_0), (S.WeightType.Q4K, o.ACT_Q8K)):
        announce(f"separate quantizer k={k} kind={kind}")
        ws = S.new_workspace(ty, 3, k)
        S.quantize_into(ty, dev(x), 3, k, ws)
        codes, d, _ = read_act(ws, kind, 3, k)
        wd, _, wcodes = o.act_quantize(kind, x, 3, k)
        assert (codes == wcodes).all()
        assert_same(d, wd)


@pytest.mark.parametrize("k,seed", ROWS)
def test_lone_q4k_gemv_quantizes_as_the_oracle(S, k, seed):
    n_out = 96
    rs = np.random.default_rng(seed)
    w = random_q4k(rs, n_out, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), n_out, k))
    for nf in (None, np.nan, np.inf):
        x = crafted_row(k, seed, nf)
        announce(f"lone q4k x8 k={k} nonfinite={nf}")
        got = host(S.gemv(W, dev(x), 1))
        want = o.gemv(o.Q4_K, w, n_out, k, x, 1, threads=8)
        assert_same(got, want, f"k {k} nonfinite {nf}")
        if nf is not None:
            assert np.isnan(got).all()


def test_gate_up_act_and_two_rows_quantize_as_the_oracle(S):
    n, k = 64, 4096
    rs = np.random.default_rng(21)
    w = random_q4k(rs, 2 * n, k)
    W = S.repack(S.Weights(S.WeightType.Q4K, dev(w), 2 * n, k))
    x = crafted_row(k, 22)
    announce("gate_up_act crafted row")
    assert_same(host(S.gate_up_act(W, dev(x), 1)), o.gate_up_act(o.Q4_K, w, n, k, x, 1, threads=8), "gate_up_act")
    x2 = np.stack([crafted_row(k, 23), crafted_row(k, 24)])
    W2 = S.repack(S.Weights(S.WeightType.Q4K, dev(w), 2 * n, k))
    announce("two-row fused decode crafted rows")
    assert_same(host(S.gemv(W2, dev(x2), 2)), o.gemv(o.Q4_K, w, 2 * n, k, x2, 2, threads=8), "two rows")


@pytest.mark.parametrize("ty", [o.Q8_0, o.Q4_0])
def test_split_one_row_quantizes_as_the_oracle(S, ty):
    n_out, k = 128, 4096
    rs = np.random.default_rng(31 + ty)
    w = o.quantize(ty, rs.standard_normal(n_out * k).astype(np.float32) * np.float32(0.02))
    W = S.repack(S.Weights(S.WeightType(ty), dev(w), n_out, k))
    for nf in (None, np.nan):
        x = crafted_row(k, 32, nf)
        announce(f"split one row ty={ty} nonfinite={nf}")
        assert_same(host(S.gemv(W, dev(x), 1)), o.gemv(ty, w, n_out, k, x, 1, threads=8), f"split {nf}")


def test_moe_gather_quantizes_as_the_oracle(S):
    import syntropy_amd.moe as M
    from test_gpu_moe import fast_q4k_experts
    s = M.MoeShape(8, 2, 4096, 512)
    gate, up, down = fast_q4k_experts(41, s.n_experts, s.hidden, s.inter)
    rows = 6
    x = np.stack([crafted_row(s.hidden, 50 + r) for r in range(rows)])
    ids = np.array([[r % 8, (r + 3) % 8] for r in range(rows)], np.int32)
    announce("moe gather crafted rows")
    out = M.moe_grouped(s, M.Experts(12, dev(gate), dev(up), dev(down)), dev(x), dev(ids))
    want = o.moe_grouped(o.Q4_K, o.Q4_K, 8, 2, 4096, 512, gate, up, down, x, ids, threads=8)
    assert_same(host(out), want, "moe")
