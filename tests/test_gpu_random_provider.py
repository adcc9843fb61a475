"""The drop-in boundary over seeded random shapes: Gemv, Gemm and GateUpAct{Silu} keys over Q4_K,
Q8_0 and Q4_0 weights, in the source layout or repacked by the provider's own `repack`, through
query -> prepare -> launch on the provider table, every output bit-identical to the oracle.

The provider sizes each op's workspace and picks its kernels from the key and the shape alone;
these cases land between the shapes its fixed tests pin."""
import ctypes as C
import json

import numpy as np
import pytest

from gpu_util import announce, assert_same, dev
from oracle import oracle as o
from test_gpu_gemm import random_q4k
from test_gpu_provider import Ctx, dense_key, shape

pytestmark = pytest.mark.gpu

OPS = ["Gemv", "Gemm", {"GateUpAct": {"act": "Silu"}}]
TYPES = [o.Q4_K, o.Q8_0, o.Q4_0]
ROWS = [1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 32, 40, 64, 65]


@pytest.fixture(scope="module")
def cx():
    c = Ctx()
    yield c
    c.close()


def draw(case: int):
    """(op, type, layout wanted, rows, n (output rows), k) of one case."""
    rs = np.random.default_rng(0x9E0A00 + case)
    op = OPS[case % len(OPS)]
    ty = TYPES[(case // len(OPS)) % len(TYPES)]
    repack = bool(rs.integers(0, 2))
    rows = int(rs.choice(ROWS))
    be = o.BLOCK_ELEMS[ty]
    if ty == o.Q4_K and repack and rows >= 32:
        k = 2048 * int(rs.integers(1, 5))  # the X8 GEMM takes rows of whole 8-block runs
    else:
        k = be * int(rs.integers(1, 8192 // be + 1))
    n = int(rs.integers(1, max(2, min(3000, (6 << 20) // k)) + 1))
    return op, ty, repack, rows, n, k


def repacked(pr, key, w):
    """The provider's repack of host bytes: (bytes, layout), or (w, 0) where it has none."""
    kb = json.dumps(key).encode()
    kbuf = (C.c_uint8 * len(kb)).from_buffer_copy(kb)
    present, layout = C.c_uint32(), C.c_uint32()
    dst = np.zeros_like(w)
    st = pr.vt.repack(pr.vt.slf, kbuf, len(kb), w.ctypes.data_as(C.POINTER(C.c_uint8)), w.size,
                      dst.ctypes.data_as(C.POINTER(C.c_uint8)), dst.size, C.byref(present), C.byref(layout))
    assert st.cls == 0
    return (dst, layout.value) if present.value else (w, 0)


@pytest.mark.parametrize("case", range(90))
def test_random_op_through_the_provider(cx, case):
    op, ty, repack, rows, n, k = draw(case)
    P, pr = cx.P, cx.pr
    gated = isinstance(op, dict)
    n_w = 2 * n if gated else n  # GateUpAct's weight stacks the gate rows, then the up rows
    rs = np.random.default_rng(0x9E0B00 + case)
    if ty == o.Q4_K:
        w = random_q4k(rs, n_w, k)
    else:
        w = o.quantize(ty, rs.normal(0.0, 0.02, n_w * k).astype(np.float32))
    x = o.normal(0x9E0C00 + case, 1.0, rows * k)
    key = dense_key(op, ty)
    wl, layout = repacked(pr, key, w) if repack else (w, 0)
    key = dense_key(op, ty, layout)
    announce(f"provider random case {case}: op={op} ty={ty} layout={layout} rows={rows} n={n} k={k}")
    caps = pr.query(cx.ctx, key, shape(rows, n, k))
    assert caps is not None
    opp = pr.prepare(cx.ctx, key, shape(rows, n, k))
    assert opp.workspace == caps["workspace"]
    wd = dev(wl)
    xb, yb = cx.put(x), cx.empty(4 * rows * n)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n])],
                     [P.view(wd.data_ptr(), wl.nbytes)], cx.workspace(opp))
    pr.launch(cx.ctx, cx.s, opp, args)
    got = cx.get(yb, np.float32, (rows, n))
    want = o.gate_up_act(ty, w, n, k, x, rows, threads=16) if gated else o.gemv(ty, w, n, k, x, rows, threads=16)
    assert_same(got, want, f"case {case}")
