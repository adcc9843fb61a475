"""rows_active from the step descriptor (crates/kernels/include/syntropy/step_desc.h:53-57; the CPU
provider's reading, crates/kernels-cpu/src/launch.rs:320-340): a launch bound to a descriptor
computes only its first rows_active rows, bit-exact, and writes nothing past them; the kernels
read the value on the device, so a captured graph follows it at every replay."""
import numpy as np
import pytest

from gpu_util import announce, assert_same, dev
from oracle import oracle as o
from refgen import GemvRng, MoeRng, gemv_activations, gemv_weights, moe_matrix
from test_gpu_provider import cx, gemv_key, shape  # noqa: F401  (the provider context fixture)

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F  # every byte of an output buffer before the launch


def step_desc(cx, rows_active):
    """A 64-byte step descriptor with rows_active at byte 8."""
    d = np.zeros(64, np.uint8)
    d[8:12] = np.frombuffer(np.uint32(rows_active).tobytes(), np.uint8)
    b = cx.put(d)
    return b, cx.P.Slice(b.handle, 0, 64)


def set_rows(cx, b, rows_active):
    d = np.zeros(64, np.uint8)
    d[8:12] = np.frombuffer(np.uint32(rows_active).tobytes(), np.uint8)
    cx.upload(b.addr, d)


def check_rows(got, want, active, what):
    """Rows below rows_active equal the oracle; the rest keep the sentinel bytes."""
    a = min(active, got.shape[0])
    if a:
        assert_same(got[:a], want[:a], what)
    rest = got[a:].view(np.uint8)
    assert (rest == SENTINEL).all(), f"{what}: rows past rows_active were written"


def dense_launch(cx, key, rows, n_out, k, w, x, step, y_cols=None):
    P, pr = cx.P, cx.pr
    y_cols = y_cols or n_out
    op = pr.prepare(cx.ctx, key, shape(rows, n_out, k))
    wd = dev(w)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * y_cols)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, y_cols])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(op), step=step)
    pr.launch(cx.ctx, cx.s, op, args)
    got = cx.get(yb, np.float32, (rows, y_cols))
    del wd
    return got


@pytest.mark.parametrize("ty,bucket,n_out,k,active", [
    (o.Q4_K, 8, 512, 2048, 5),    # the grouped-row kernel
    (o.Q8_0, 12, 300, 1024, 9),   # two 8-row launches, the second with one active row
    (o.Q4_K, 1, 1024, 4096, 0),   # single-row decode, nothing active
    (o.Q4_K, 1, 1024, 4096, 1),
    (o.Q4_K, 64, 256, 4096, 40),  # the matrix-core GEMM
    (o.Q4_K, 64, 256, 4096, 100),  # more than the bucket: the bucket
    (o.F16, 6, 100, 256, 3)])
def test_gemv_rows_active(cx, ty, bucket, n_out, k, active):
    rng = GemvRng(ty * 100 + bucket * 7 + active)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, bucket, k).reshape(bucket, k)
    _, step = step_desc(cx, active)
    announce(f"rows_active gemv ty={ty} bucket={bucket} active={active}")
    key = gemv_key(ty) if ty != o.F16 else {"op": "Gemv", "schemes": [{"Plain": "F16"}, {"Plain": "F32"},
                                                                      {"Plain": "F32"}], "layout": 0, "variant": 0}
    got = dense_launch(cx, key, bucket, n_out, k, w, x, step)
    a = min(active, bucket)
    want = o.gemv(ty, w, n_out, k, x[:a], a, threads=8) if a else None
    check_rows(got, want, active, f"gemv ty={ty}")


@pytest.mark.parametrize("bucket,n_out,active", [(1, 1024, 0), (1, 1024, 1), (2, 1024, 0), (2, 1024, 1),
                                                 (3, 8200, 2), (3, 8200, 3)])
def test_x8_rows_active(cx, bucket, n_out, active):
    """X8 weights at one row (the fused decode kernel) and at two and three rows (the decode
    kernel over rows side by side in LDS), with fewer rows active than the bucket."""
    import ctypes as C
    import json
    P, pr = cx.P, cx.pr
    rng = GemvRng(991 + bucket)
    k = 4096
    w = gemv_weights(rng, o.Q4_K, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, bucket, k).reshape(bucket, k)
    kb = json.dumps(gemv_key(o.Q4_K)).encode()
    kbuf = (C.c_uint8 * len(kb)).from_buffer_copy(kb)
    present, lay = C.c_uint32(), C.c_uint32()
    wl = np.zeros_like(w)
    pr.vt.repack(pr.vt.slf, kbuf, len(kb), w.ctypes.data_as(C.POINTER(C.c_uint8)), w.size,
                 wl.ctypes.data_as(C.POINTER(C.c_uint8)), wl.size, C.byref(present), C.byref(lay))
    _, step = step_desc(cx, active)
    announce(f"rows_active x8 bucket={bucket} n_out={n_out} active={active}")
    got = dense_launch(cx, dict(gemv_key(o.Q4_K), layout=1), bucket, n_out, k, wl, x, step)
    a = min(active, bucket)
    want = o.gemv(o.Q4_K, w, n_out, k, x[:a], a, threads=8) if a else None
    check_rows(got, want, active, "x8")


@pytest.mark.parametrize("ty,bucket,active", [(o.Q8_0, 1, 0), (o.Q8_0, 1, 1), (o.Q4_0, 1, 1), (o.Q8_0, 12, 9),
                                              (o.Q8_0, 40, 17), (o.Q8_0, 40, 3), (o.Q4_0, 12, 10), (o.Q4_0, 40, 33),
                                              (o.Q4_0, 40, 0)])
def test_split_layout_rows_active(cx, ty, bucket, active):
    """Layout 2 (SPLIT): the split decode kernel quantizing its one row in its workgroups, the
    K-split int8 GEMM (twelve rows) and the staged int8 GEMM (forty rows)."""
    import ctypes as C
    import json
    P, pr = cx.P, cx.pr
    rng = GemvRng(77 * ty + bucket + active)
    n_out, k = 200, 1024
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, bucket, k).reshape(bucket, k)
    kb = json.dumps(gemv_key(ty)).encode()
    kbuf = (C.c_uint8 * len(kb)).from_buffer_copy(kb)
    present, lay = C.c_uint32(), C.c_uint32()
    wl = np.zeros_like(w)
    pr.vt.repack(pr.vt.slf, kbuf, len(kb), w.ctypes.data_as(C.POINTER(C.c_uint8)), w.size,
                 wl.ctypes.data_as(C.POINTER(C.c_uint8)), wl.size, C.byref(present), C.byref(lay))
    assert lay.value == 2
    _, step = step_desc(cx, active)
    announce(f"rows_active split ty={ty} bucket={bucket} active={active}")
    got = dense_launch(cx, dict(gemv_key(ty), layout=2), bucket, n_out, k, wl, x, step)
    a = min(active, bucket)
    want = o.gemv(ty, w, n_out, k, x[:a], a, threads=8) if a else None
    check_rows(got, want, active, f"split ty={ty}")


def test_gate_up_act_rows_active(cx):
    rng = GemvRng(515)
    n, k, bucket, active = 300, 1024, 4, 2
    w = gemv_weights(rng, o.Q4_K, 2 * n, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, bucket, k).reshape(bucket, k)
    _, step = step_desc(cx, active)
    key = dict(gemv_key(o.Q4_K), op={"GateUpAct": {"act": "Silu"}})
    announce("rows_active gate_up_act")
    got = dense_launch(cx, key, bucket, n, k, w, x, step)
    check_rows(got, o.gate_up_act(o.Q4_K, w, n, k, x[:active], active, threads=8), active, "gate_up_act")


@pytest.mark.parametrize("E,top_k,hidden,inter,bucket,active", [
    (16, 4, 512, 256, 16, 9),      # decode kernels
    (6, 2, 256, 512, 300, 200)])   # the many-token GEMM path
def test_moe_rows_active(cx, E, top_k, hidden, inter, bucket, active):
    """Route, grouped FFN and combine bound to one descriptor.  The inactive rows' ids are out of
    range: the grouped FFN must not read them (no error), and no output past rows_active moves."""
    P, pr = cx.P, cx.pr
    rng = MoeRng(E * 1000 + bucket)
    gate = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
    up = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
    down = moe_matrix(rng, o.Q4_K, E * hidden, inter, o.f16_bits)
    router = o.normal(0x51A30004 + E, 0.02, E * hidden).reshape(E, hidden)
    x = o.normal(0x51A20004 + bucket, 1.0, bucket * hidden).reshape(bucket, hidden)
    _, step = step_desc(cx, active)
    announce(f"rows_active moe E={E} bucket={bucket} active={active}")
    route_key = {"op": {"MoeRoute": {"norm": "Softmax"}}, "schemes": [{"Plain": "F32"}, {"Plain": "F32"}],
                 "layout": 0, "variant": 0}
    grouped_key = {"op": "MoeGrouped", "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}],
                   "layout": 0, "variant": 0}
    combine_key = {"op": "MoeCombine", "schemes": [{"Plain": "F32"}], "layout": 0, "variant": 0}
    r_op = pr.prepare(cx.ctx, route_key, shape(bucket, E, top_k, hidden))
    g_op = pr.prepare(cx.ctx, grouped_key, shape(bucket, E, top_k, hidden, inter))
    c_op = pr.prepare(cx.ctx, combine_key, shape(bucket, top_k, 0, hidden))
    rd, gd, ud, dd = dev(router), dev(gate), dev(up), dev(down)
    xb = cx.put(x)
    ids0 = np.full((bucket, top_k), 999, np.int32)  # out of range past rows_active
    ids_b, w_b = cx.put(ids0), cx.empty(4 * bucket * top_k)
    per_b, y_b = cx.empty(4 * bucket * top_k * hidden), cx.empty(4 * bucket * hidden)
    x_arg = P.packed(xb, P.DT_F32, [bucket, hidden])
    ids_arg = P.packed(ids_b, P.DT_I32, [bucket, top_k])
    w_arg = P.packed(w_b, P.DT_F32, [bucket, top_k])
    per_arg = P.packed(per_b, P.DT_F32, [bucket, top_k, hidden])
    y_arg = P.packed(y_b, P.DT_F32, [bucket, hidden])
    pr.launch(cx.ctx, cx.s, r_op, P.op_args([x_arg], [ids_arg, w_arg], [P.view(rd.data_ptr(), router.nbytes)],
                                            cx.workspace(r_op), [P.Scalar(1, 1)], step=step))
    views = [P.view(t.data_ptr(), t.numel()) for t in (gd, ud, dd)]
    pr.launch(cx.ctx, cx.s, g_op, P.op_args([x_arg, ids_arg], [per_arg], views, cx.workspace(g_op), step=step))
    pr.launch(cx.ctx, cx.s, c_op, P.op_args([per_arg, w_arg], [y_arg], [], step=step))

    xa = x[:active]
    wids, ww, _ = o.moe_route(router, xa, E, top_k, True)
    ids = cx.get(ids_b, np.int32, (bucket, top_k))
    assert (ids[:active] == wids).all() and (ids[active:] == 999).all()
    check_rows(cx.get(w_b, np.float32, (bucket, top_k)), ww, active, "route weights")
    want_per = o.moe_grouped(o.Q4_K, o.Q4_K, E, top_k, hidden, inter, gate, up, down, xa, wids, threads=8)
    per = cx.get(per_b, np.float32, (bucket, top_k * hidden))
    check_rows(per, want_per.reshape(active, top_k * hidden), active, "grouped")
    want_y = o.moe_combine_ranked(want_per.reshape(active, top_k, hidden), ww)
    check_rows(cx.get(y_b, np.float32, (bucket, hidden)), want_y, active, "combine")


def test_captured_graph_follows_rows_active(cx):
    """One capture, replayed with rows_active 8, 3 and 0 written into the descriptor between
    replays (and the output reset), each replay computing exactly that many rows."""
    P, pr = cx.P, cx.pr
    bucket, n_out, k = 8, 384, 2048
    rng = GemvRng(8383)
    w = gemv_weights(rng, o.Q4_K, n_out, k, o.f16_bits, o.round_bf16)
    op = pr.prepare(cx.ctx, gemv_key(o.Q4_K), shape(bucket, n_out, k))
    wd = dev(w)
    xb, yb = cx.empty(4 * bucket * k, 0), cx.empty(4 * bucket * n_out)
    db, step = step_desc(cx, bucket)
    args = P.op_args([P.packed(xb, P.DT_F32, [bucket, k])], [P.packed(yb, P.DT_F32, [bucket, n_out])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(op), step=step)
    announce("rows_active capture/replay")
    pr.begin_capture(cx.ctx, cx.s)
    pr.launch(cx.ctx, cx.s, op, args)
    g = pr.end_capture(cx.ctx, cx.s)
    for active in (8, 3, 0):
        x = gemv_activations(rng, bucket, k).reshape(bucket, k).astype(np.float32)
        cx.upload(xb.addr, x)
        cx.upload(yb.addr, np.full(4 * bucket * n_out, SENTINEL, np.uint8))
        set_rows(cx, db, active)
        pr.replay(cx.ctx, cx.s, g)
        got = cx.get(yb, np.float32, (bucket, n_out))
        want = o.gemv(o.Q4_K, w, n_out, k, x[:active], active, threads=8) if active else None
        check_rows(got, want, active, f"replay rows_active={active}")
