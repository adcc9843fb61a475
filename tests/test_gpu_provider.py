"""GPU parity through the provider-library boundary: the core's calling sequence (open, stream,
alloc, query, prepare, launch, synchronize) on the hip provider, each op's outputs bit-exact
against the oracle; stream capture and replay; the workspace and argument checks.

The sequence is kernels_loader::ModuleProvider's (crates/kernels-loader/src/provider.rs) and the
argument binding is the executor's (crates/kernels/src/op/args.rs:85-96: packed tensors, weight
views, the workspace slice)."""
import ctypes as C
import json

import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, require_gpu
from oracle import oracle as o
from refgen import GemvRng, MoeRng, gemv_activations, gemv_weights, moe_matrix

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class Ctx:
    """One open context and a stream; host data moves in and out with hipMemcpy."""

    def __init__(self):
        require_gpu()
        from syntropy_amd import provider as P
        self.P = P
        self.pr = P.Provider()
        self.hip = C.CDLL("libamdhip64.so.7")  # the runtime torch and the provider already share
        self.hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.hip.hipMemcpy.restype = C.c_int
        self.hip.hipDeviceSynchronize.restype = C.c_int
        self.ctx = self.pr.open(0)
        self.s = self.pr.stream(self.ctx)
        self.bufs = []

    def upload(self, addr: int, a):
        """A host-to-device copy complete before the provider's stream runs again."""
        assert self.hip.hipMemcpy(addr, a.ctypes.data, a.nbytes, H2D) == 0
        assert self.hip.hipDeviceSynchronize() == 0

    def put(self, a) -> "object":
        a = np.ascontiguousarray(a)
        b = self.pr.alloc(self.ctx, max(a.nbytes, 1))
        if a.nbytes:
            self.upload(b.addr, a)
        self.bufs.append(b)
        return b

    def empty(self, nbytes: int, fill: int = 0x7F):
        return self.put(np.full(nbytes, fill, np.uint8))

    def get(self, b, dtype, shape):
        self.pr.synchronize(self.ctx, self.s)
        out = np.empty(shape, dtype)
        assert self.hip.hipMemcpy(out.ctypes.data, b.addr, out.nbytes, D2H) == 0
        return out

    def workspace(self, op):
        if op.workspace == 0:
            return None
        ws = self.empty(op.workspace, 0)
        return self.P.Slice(ws.handle, 0, op.workspace)

    def close(self):
        self.pr.close(self.ctx)


@pytest.fixture(scope="module")
def cx():
    c = Ctx()
    yield c
    c.close()


def gemv_key(ty):
    name = {o.Q4_K: "Q4_K", o.Q8_0: "Q8_0", o.Q4_0: "Q4_0"}[ty]
    return {"op": "Gemv", "schemes": [{"Ggml": name}, {"Plain": "F32"}, {"Plain": "F32"}], "layout": 0,
            "variant": 0}


def shape(rows, *dims, cls="Decode"):
    return {"class": cls, "rows": rows, "dims": list(dims)}


@pytest.mark.parametrize("ty,rows,n_out,k", [(o.Q4_K, 1, 4096, 4096), (o.Q4_K, 7, 1536, 2048),
                                             (o.Q8_0, 3, 1000, 4096), (o.Q4_0, 2, 513, 1024)])
def test_gemv_through_the_provider(cx, ty, rows, n_out, k):
    P, pr = cx.P, cx.pr
    rng = GemvRng(ty * 1000 + rows)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    announce(f"provider gemv ty={ty} rows={rows} n_out={n_out} k={k}")
    caps = pr.query(cx.ctx, gemv_key(ty), shape(rows, n_out, k))
    assert caps is not None and caps["deterministic"] and caps["capture_safe"]
    op = pr.prepare(cx.ctx, gemv_key(ty), shape(rows, n_out, k))
    assert op.workspace == caps["workspace"]
    wd = dev(w)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * n_out)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n_out])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(op))
    pr.launch(cx.ctx, cx.s, op, args)
    got = cx.get(yb, np.float32, (rows, n_out))
    assert_same(got, o.gemv(ty, w, n_out, k, x, rows, threads=8), "provider gemv")


@pytest.mark.parametrize("ty,rows,n_out,k,want_layout", [
    (o.Q4_K, 1, 4096, 4096, 1), (o.Q4_K, 1, 1000, 14336, 1), (o.Q4_K, 64, 256, 4096, 1),
    (o.Q8_0, 1, 4096, 4096, 2), (o.Q8_0, 5, 1000, 14336, 2), (o.Q8_0, 40, 300, 4096, 2),
    (o.Q4_0, 1, 4096, 4096, 2), (o.Q4_0, 11, 513, 1024, 2)])
def test_gemv_repacked_layout_through_the_provider(cx, ty, rows, n_out, k, want_layout):
    """The core's path for repacked weights: repacked_len / repack on the host bytes (Q4_K to
    layout 1, Q8_0 and Q4_0 to layout 2), then the Gemv key with the layout repack returned;
    outputs equal the oracle on the source bytes."""
    P, pr = cx.P, cx.pr
    rng = GemvRng(rows * 7 + n_out + ty)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    src_key = gemv_key(ty)
    kb = json.dumps(src_key).encode()
    kbuf = (C.c_uint8 * len(kb)).from_buffer_copy(kb)
    present, layout = C.c_uint32(), C.c_uint32()
    dst = np.zeros_like(w)
    st = pr.vt.repack(pr.vt.slf, kbuf, len(kb), w.ctypes.data_as(C.POINTER(C.c_uint8)), w.size,
                      dst.ctypes.data_as(C.POINTER(C.c_uint8)), dst.size, C.byref(present), C.byref(layout))
    assert st.cls == 0 and (present.value, layout.value) == (1, want_layout)
    key = dict(src_key, layout=layout.value)
    announce(f"provider gemv layout {want_layout} ty={ty} rows={rows} n_out={n_out} k={k}")
    caps = pr.query(cx.ctx, key, shape(rows, n_out, k))
    assert caps is not None and caps["layout"] == want_layout
    op = pr.prepare(cx.ctx, key, shape(rows, n_out, k))
    wd = dev(dst)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * n_out)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n_out])],
                     [P.view(wd.data_ptr(), dst.nbytes)], cx.workspace(op))
    pr.launch(cx.ctx, cx.s, op, args)
    got = cx.get(yb, np.float32, (rows, n_out))
    assert_same(got, o.gemv(ty, w, n_out, k, x, rows, threads=8), f"provider gemv layout {want_layout}")


def dense_key(op, ty, layout=0):
    return dict(gemv_key(ty), op=op, layout=layout)


@pytest.mark.parametrize("op,ty,rows,n_out,k", [
    ("Gemm", o.Q4_K, 64, 512, 4096), ("Gemm", o.Q8_0, 20, 300, 1024),
    ("Logits", o.Q4_K, 1, 3000, 2048), ("Logits", o.Q4_0, 2, 777, 512)])
def test_gemm_and_logits_keys_take_the_gemv_binding(cx, op, ty, rows, n_out, k):
    """Gemm and Logits are matrix products with Gemv's operands (the ggml provider maps all three
    to mul_mat, crates/kernels-ggml/src/mapping.rs:30); their values are Gemv's."""
    P, pr = cx.P, cx.pr
    rng = GemvRng(ty * 77 + rows)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    announce(f"provider {op} ty={ty} rows={rows} n_out={n_out} k={k}")
    key = dense_key(op, ty)
    assert pr.query(cx.ctx, key, shape(rows, n_out, k)) is not None
    opp = pr.prepare(cx.ctx, key, shape(rows, n_out, k))
    wd = dev(w)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * n_out)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n_out])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(opp))
    pr.launch(cx.ctx, cx.s, opp, args)
    assert_same(cx.get(yb, np.float32, (rows, n_out)), o.gemv(ty, w, n_out, k, x, rows, threads=8), op)


@pytest.mark.parametrize("ty,rows,n,k,layout", [(o.Q4_K, 1, 1536, 4096, 0), (o.Q4_K, 40, 512, 2048, 0),
                                                (o.Q4_K, 1, 1024, 4096, 1), (o.Q8_0, 3, 700, 1024, 0),
                                                (o.Q4_0, 1, 256, 512, 0), (o.Q8_0, 1, 700, 1024, 2),
                                                (o.Q8_0, 12, 300, 2048, 2), (o.Q4_0, 4, 256, 512, 2)])
def test_gate_up_act_through_the_provider(cx, ty, rows, n, k, layout):
    """GateUpAct{Silu}: one weight of 2 n rows, gate then up (mapping.rs:31); y [rows, n]."""
    P, pr = cx.P, cx.pr
    rng = GemvRng(ty * 55 + rows + n)
    w = gemv_weights(rng, ty, 2 * n, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    wl = w
    if layout:
        wl = np.zeros_like(w)
        kb = json.dumps(dense_key({"GateUpAct": {"act": "Silu"}}, ty)).encode()
        kbuf = (C.c_uint8 * len(kb)).from_buffer_copy(kb)
        present, lay = C.c_uint32(), C.c_uint32()
        st = pr.vt.repack(pr.vt.slf, kbuf, len(kb), w.ctypes.data_as(C.POINTER(C.c_uint8)), w.size,
                          wl.ctypes.data_as(C.POINTER(C.c_uint8)), wl.size, C.byref(present), C.byref(lay))
        assert st.cls == 0 and (present.value, lay.value) == (1, layout)
    key = dense_key({"GateUpAct": {"act": "Silu"}}, ty, layout)
    announce(f"provider gate_up_act ty={ty} rows={rows} n={n} k={k} layout={layout}")
    assert pr.query(cx.ctx, key, shape(rows, n, k)) is not None
    opp = pr.prepare(cx.ctx, key, shape(rows, n, k))
    wd = dev(wl)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * n)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n])],
                     [P.view(wd.data_ptr(), wl.nbytes)], cx.workspace(opp))
    pr.launch(cx.ctx, cx.s, opp, args)
    assert_same(cx.get(yb, np.float32, (rows, n)), o.gate_up_act(ty, w, n, k, x, rows, threads=8), "gate_up_act")


@pytest.mark.parametrize("scheme,ty", [({"Plain": "F16"}, o.F16), ({"Ggml": "BF16"}, o.BF16)])
def test_float_gemv_through_the_provider(cx, scheme, ty):
    """Plain and GGUF F16/BF16 weights (gemv/entry.rs:41-47): F32 accumulation, no workspace
    beyond the alignment slack, no activation quantization."""
    P, pr = cx.P, cx.pr
    rows, n_out, k = 2, 777, 1024
    rng = GemvRng(ty * 13)
    w = gemv_weights(rng, ty, n_out, k, o.f16_bits, o.round_bf16)
    x = gemv_activations(rng, rows, k)
    key = {"op": "Gemv", "schemes": [scheme, {"Plain": "F32"}, {"Plain": "F32"}], "layout": 0, "variant": 0}
    caps = pr.query(cx.ctx, key, shape(rows, n_out, k))
    assert caps is not None and caps["numerics"]["accumulate"] == 0 and caps["numerics"]["act_in"] == 0
    announce(f"provider float gemv {scheme}")
    op = pr.prepare(cx.ctx, key, shape(rows, n_out, k))
    wd = dev(w)
    xb, yb = cx.put(x.astype(np.float32)), cx.empty(4 * rows * n_out)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n_out])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(op))
    pr.launch(cx.ctx, cx.s, op, args)
    assert_same(cx.get(yb, np.float32, (rows, n_out)), o.gemv(ty, w, n_out, k, x, rows, threads=8), "float")


def test_query_answers_none_for_unserved_shapes(cx):
    pr = cx.pr
    assert pr.query(cx.ctx, gemv_key(o.Q4_K), shape(1, 64, 100)) is None  # k not whole super-blocks
    key = dict(gemv_key(o.Q4_K), schemes=[{"Ggml": "Q6_K"}, {"Plain": "F32"}, {"Plain": "F32"}])
    assert pr.query(cx.ctx, key, shape(1, 64, 256)) is None
    assert pr.query(cx.ctx, dict(gemv_key(o.Q4_K), layout=3), shape(1, 64, 256)) is None
    gelu = dense_key({"GateUpAct": {"act": "Gelu"}}, o.Q4_K)
    assert pr.query(cx.ctx, gelu, shape(1, 64, 256)) is None  # no reference form of GELU gating
    assert pr.query(cx.ctx, dict(gemv_key(o.Q8_0), layout=1), shape(1, 64, 256)) is None
    assert pr.query(cx.ctx, dict(gemv_key(o.Q4_K), layout=2), shape(1, 64, 256)) is None
    assert pr.query(cx.ctx, dict(gemv_key(o.Q8_0), layout=2), shape(130, 64, 256)) is not None
    assert pr.query(cx.ctx, dict(gemv_key(o.Q4_K), layout=1), shape(32, 64, 1536)) is None  # GEMM: k % 2048
    assert pr.query(cx.ctx, dict(gemv_key(o.Q4_K), layout=1), shape(31, 64, 1536)) is not None  # 2..31 rows
    assert pr.query(cx.ctx, {"op": "Attention", "schemes": [], "layout": 0, "variant": 0},
                    shape(1, 64, 256)) is None
    with pytest.raises(cx.P.ProviderError) as e:
        pr.prepare(cx.ctx, gemv_key(o.Q4_K), shape(1, 64, 100))
    assert (e.value.cls, e.value.code) == (2, 1)


def test_launch_checks_workspace_and_arguments(cx):
    P, pr = cx.P, cx.pr
    rows, n_out, k = 2, 256, 512
    op = pr.prepare(cx.ctx, gemv_key(o.Q4_K), shape(rows, n_out, k))
    w = torch.zeros(n_out * k // 256 * 144, dtype=torch.uint8, device="cuda")
    xb, yb = cx.empty(4 * rows * k, 0), cx.empty(4 * rows * n_out)
    small = cx.empty(64, 0)
    announce("provider launch refusals")
    x_arg, y_arg = P.packed(xb, P.DT_F32, [rows, k]), P.packed(yb, P.DT_F32, [rows, n_out])
    wv = [P.view(w.data_ptr(), w.numel())]
    with pytest.raises(P.ProviderError) as e:
        pr.launch(cx.ctx, cx.s, op, P.op_args([x_arg], [y_arg], wv, P.Slice(small.handle, 0, 64)))
    assert (e.value.cls, e.value.code) == (13, 14)
    ws = cx.workspace(op)
    with pytest.raises(P.ProviderError) as e:  # dims not the plan's
        pr.launch(cx.ctx, cx.s, op, P.op_args([P.packed(xb, P.DT_F32, [rows, k // 2])], [y_arg], wv, ws))
    assert "dims" in e.value.message
    with pytest.raises(P.ProviderError) as e:  # a short weight view
        pr.launch(cx.ctx, cx.s, op, P.op_args([x_arg], [y_arg], [P.view(w.data_ptr(), 100)], ws))
    assert "weight view" in e.value.message
    # nothing was written by the refused launches
    assert (cx.get(yb, np.uint8, 4 * rows * n_out) == 0x7F).all()


def fast_q4k_experts(seed, n_experts, hidden, inter):
    """Stacked Q4_K experts: random codes, F16 scales in [2^-10, 2^-5) (the distribution of
    crates/kernels-cpu/src/moe/tests.rs:40-74, generated vectorized for the layer-size case)."""
    rs = np.random.default_rng(seed)

    def mat(n_out, k):
        nb = n_out * k // 256
        b = np.frombuffer(rs.bytes(nb * 144), np.uint8).reshape(nb, 144).copy()
        h = ((rs.integers(5, 10, (nb, 2), dtype=np.uint16) << 10)
             | rs.integers(0, 1024, (nb, 2), dtype=np.uint16)).astype(np.uint16)
        b[:, 0:4] = h.view(np.uint8).reshape(nb, 4)
        return b.ravel()

    return mat(n_experts * inter, hidden), mat(n_experts * inter, hidden), mat(n_experts * hidden, inter)


@pytest.mark.parametrize("E,top_k,hidden,inter,rows,n_shared", [
    (16, 4, 512, 256, 37, 2),
    (128, 8, 4096, 1536, 64, 0)])  # the Qwen3-235B-A22B MoE shape at 64 decode tokens
def test_moe_layer_through_the_provider(cx, E, top_k, hidden, inter, rows, n_shared):
    """Route, grouped experts, combine: three prepared ops on one stream under the reference's
    keys and bindings (MoeCombine: dims [top_k, n_shared, hidden], inputs [per_expert, weights,
    shared...], crates/kernels/src/op/kind.rs:244, crates/graph/src/blocks/ffn.rs:189-200), every
    output bit-exact."""
    P, pr = cx.P, cx.pr
    if E == 128:
        gate, up, down = fast_q4k_experts(7, E, hidden, inter)
    else:
        rng = MoeRng(77)
        gate = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
        up = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
        down = moe_matrix(rng, o.Q4_K, E * hidden, inter, o.f16_bits)
    router = o.normal(0x51A30004, 0.02, E * hidden).reshape(E, hidden)
    x = o.normal(0x51A20004, 1.0, rows * hidden).reshape(rows, hidden)
    shared = [o.normal(0x51A50000 + i, 1.0, rows * hidden).reshape(rows, hidden) for i in range(n_shared)]
    announce(f"provider moe E={E} k={top_k} hidden={hidden} inter={inter} rows={rows} shared={n_shared}")

    route_key = {"op": {"MoeRoute": {"norm": "Softmax"}}, "schemes": [{"Plain": "F32"}, {"Plain": "F32"}],
                 "layout": 0, "variant": 0}
    grouped_key = {"op": "MoeGrouped", "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}],
                   "layout": 0, "variant": 0}
    combine_key = {"op": "MoeCombine", "schemes": [{"Plain": "F32"}], "layout": 0, "variant": 0}
    caps = pr.query(cx.ctx, route_key, shape(rows, E, top_k, hidden))
    assert caps["numerics"]["softmax_f32"]
    ccaps = pr.query(cx.ctx, combine_key, shape(rows, top_k, n_shared, hidden))
    assert ccaps["workspace"] == 0 and ccaps["deterministic"]
    r_op = pr.prepare(cx.ctx, route_key, shape(rows, E, top_k, hidden))
    g_op = pr.prepare(cx.ctx, grouped_key, shape(rows, E, top_k, hidden, inter))
    c_op = pr.prepare(cx.ctx, combine_key, shape(rows, top_k, n_shared, hidden))

    rd, gd, ud, dd = dev(router), dev(gate), dev(up), dev(down)
    xb = cx.put(x)
    ids_b, w_b = cx.empty(4 * rows * top_k), cx.empty(4 * rows * top_k)
    per_b, y_b = cx.empty(4 * rows * top_k * hidden), cx.empty(4 * rows * hidden)
    x_arg = P.packed(xb, P.DT_F32, [rows, hidden])
    ids_arg = P.packed(ids_b, P.DT_I32, [rows, top_k])
    w_arg = P.packed(w_b, P.DT_F32, [rows, top_k])
    per_arg = P.packed(per_b, P.DT_F32, [rows, top_k, hidden])
    y_arg = P.packed(y_b, P.DT_F32, [rows, hidden])
    sh_args = [P.packed(cx.put(a), P.DT_F32, [rows, hidden]) for a in shared]
    pr.launch(cx.ctx, cx.s, r_op, P.op_args([x_arg], [ids_arg, w_arg], [P.view(rd.data_ptr(), router.nbytes)],
                                            cx.workspace(r_op), [P.Scalar(1, 1)]))
    views = [P.view(t.data_ptr(), t.numel()) for t in (gd, ud, dd)]
    pr.launch(cx.ctx, cx.s, g_op, P.op_args([x_arg, ids_arg], [per_arg], views, cx.workspace(g_op)))
    pr.launch(cx.ctx, cx.s, c_op, P.op_args([per_arg, w_arg, *sh_args], [y_arg], []))

    wids, ww, _ = o.moe_route(router, x, E, top_k, True)
    assert (cx.get(ids_b, np.int32, (rows, top_k)) == wids).all()
    assert_same(cx.get(w_b, np.float32, (rows, top_k)), ww, "route weights")
    want = o.moe_grouped(o.Q4_K, o.Q4_K, E, top_k, hidden, inter, gate, up, down, x, wids, threads=16)
    assert_same(cx.get(per_b, np.float32, (rows, top_k, hidden)), want, "grouped")
    assert_same(cx.get(y_b, np.float32, (rows, hidden)), o.moe_combine_ranked(want, ww, shared), "combined")
    del gd, ud, dd
    torch.cuda.empty_cache()


def test_moe_combine_binding_refusals(cx):
    """MoeCombine's query answers None for shapes outside [top_k 1..64, n_shared 0..8, hidden];
    a launch with a shared-output count other than the plan's is refused."""
    P, pr = cx.P, cx.pr
    key = {"op": "MoeCombine", "schemes": [{"Plain": "F32"}], "layout": 0, "variant": 0}
    for dims in ([0, 0, 64], [65, 0, 64], [2, 9, 64], [2, 0, 0], [2, 64], [2, 0, 64, 1]):
        assert pr.query(cx.ctx, key, shape(4, *dims)) is None, dims
    assert pr.query(cx.ctx, key, shape(4, 2, 0, 64)) is not None  # the ggml mapping test's key
    rows, top_k, hidden = 4, 2, 64
    op = pr.prepare(cx.ctx, key, shape(rows, top_k, 1, hidden))
    per = P.packed(cx.empty(4 * rows * top_k * hidden), P.DT_F32, [rows, top_k, hidden])
    w = P.packed(cx.empty(4 * rows * top_k), P.DT_F32, [rows, top_k])
    yb = cx.empty(4 * rows * hidden)
    y = P.packed(yb, P.DT_F32, [rows, hidden])
    with pytest.raises(P.ProviderError) as e:
        pr.launch(cx.ctx, cx.s, op, P.op_args([per, w], [y], []))
    assert "shared" in e.value.message
    assert (cx.get(yb, np.uint8, 4 * rows * hidden) == 0x7F).all()


def test_moe_grouped_site_input_through_the_provider(cx):
    """MoeGrouped's input 2, packed I32 [n_experts, 1] (crates/kernels-cpu/src/moe/entry.rs:13-16,
    158-160): a zero leaves the expert's slots as they were."""
    P, pr = cx.P, cx.pr
    E, top_k, hidden, inter, rows = 8, 2, 256, 512, 5
    rng = MoeRng(78)
    gate = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
    up = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
    down = moe_matrix(rng, o.Q4_K, E * hidden, inter, o.f16_bits)
    x = o.normal(0x51A20005, 1.0, rows * hidden).reshape(rows, hidden)
    ids = np.array([[0, 1], [2, 3], [4, 5], [6, 7], [1, 6]], np.int32)
    site = np.array([1, 0, 1, 1, 0, 0, 1, 0], np.int32)
    announce(f"provider moe site E={E} rows={rows}")
    key = {"op": "MoeGrouped", "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}],
           "layout": 0, "variant": 0}
    op = pr.prepare(cx.ctx, key, shape(rows, E, top_k, hidden, inter))
    gd, ud, dd = dev(gate), dev(up), dev(down)
    xb, ib, sb = cx.put(x), cx.put(ids), cx.put(site)
    per_b = cx.put(np.full(rows * top_k * hidden, 0x7FC0DEAD, np.uint32))
    views = [P.view(t.data_ptr(), t.numel()) for t in (gd, ud, dd)]
    ins = [P.packed(xb, P.DT_F32, [rows, hidden]), P.packed(ib, P.DT_I32, [rows, top_k])]
    per_arg = P.packed(per_b, P.DT_F32, [rows, top_k, hidden])
    # a site tensor of the wrong shape is refused before anything runs
    with pytest.raises(P.ProviderError):
        pr.launch(cx.ctx, cx.s, op, P.op_args(ins + [P.packed(sb, P.DT_I32, [E - 1, 1])], [per_arg], views,
                                              cx.workspace(op)))
    pr.launch(cx.ctx, cx.s, op, P.op_args(ins + [P.packed(sb, P.DT_I32, [E, 1])], [per_arg], views,
                                          cx.workspace(op)))
    want = o.moe_grouped(o.Q4_K, o.Q4_K, E, top_k, hidden, inter, gate, up, down, x, ids, site=site,
                         out=np.full(rows * top_k * hidden, 0x7FC0DEAD, np.uint32).view(np.float32))
    got = cx.get(per_b, np.float32, (rows, top_k, hidden))
    assert_same(got, want, "site")
    assert (got[site[ids] == 0].view(np.uint32) == 0x7FC0DEAD).all()


@pytest.mark.parametrize("rows", [5, 120])
def test_moe_grouped_refusal_is_reported_at_synchronize(rows):
    """An id naming no expert: the launch writes nothing (the decode kernels at 5 rows, the
    many-token path at 120), and the next synchronize reports the first such slot as Internal,
    with the CPU provider's message (crates/kernels-cpu/src/moe.rs:433-441, moe/entry.rs:309);
    the report is given once, and a clean launch after it runs."""
    c = Ctx()
    try:
        P, pr = c.P, c.pr
        E, top_k, hidden, inter = 6, 2, 256, 512
        rng = MoeRng(79)
        gate = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
        up = moe_matrix(rng, o.Q4_K, E * inter, hidden, o.f16_bits)
        down = moe_matrix(rng, o.Q4_K, E * hidden, inter, o.f16_bits)
        x = o.normal(0x51A20006, 1.0, rows * hidden).reshape(rows, hidden)
        ids = np.stack([np.arange(top_k) + r % (E - 1) for r in range(rows)]).astype(np.int32)
        bad = ids.copy()
        bad[rows - 2, 1] = E  # and a later one, which is not the first
        bad[rows - 1, 0] = -3
        key = {"op": "MoeGrouped", "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}],
               "layout": 0, "variant": 0}
        op = pr.prepare(c.ctx, key, shape(rows, E, top_k, hidden, inter))
        gd, ud, dd = dev(gate), dev(up), dev(down)
        views = [P.view(t.data_ptr(), t.numel()) for t in (gd, ud, dd)]
        xb, bb, ib = c.put(x), c.put(bad), c.put(ids)
        per_b = c.put(np.full(rows * top_k * hidden, 0x7FC0DEAD, np.uint32))
        per_arg = P.packed(per_b, P.DT_F32, [rows, top_k, hidden])
        ws = c.workspace(op)
        announce(f"provider moe refusal rows={rows}")
        pr.launch(c.ctx, c.s, op, P.op_args([P.packed(xb, P.DT_F32, [rows, hidden]),
                                             P.packed(bb, P.DT_I32, [rows, top_k])], [per_arg], views, ws))
        with pytest.raises(P.ProviderError) as e:
            pr.synchronize(c.ctx, c.s)
        assert e.value.cls == P.CLASS_INTERNAL
        assert f"row {rows - 2} rank 1 routes to expert {E}" in e.value.message, e.value.message
        assert any(f"routes to expert {E}" in m for _, _, m in P.LOG)
        assert (c.get(per_b, np.uint32, rows * top_k * hidden) == 0x7FC0DEAD).all()
        pr.synchronize(c.ctx, c.s)  # reported once
        pr.launch(c.ctx, c.s, op, P.op_args([P.packed(xb, P.DT_F32, [rows, hidden]),
                                             P.packed(ib, P.DT_I32, [rows, top_k])], [per_arg], views, ws))
        pr.synchronize(c.ctx, c.s)
        want = o.moe_grouped(o.Q4_K, o.Q4_K, E, top_k, hidden, inter, gate, up, down, x, ids, threads=8)
        assert_same(c.get(per_b, np.float32, (rows, top_k, hidden)), want, "after the refusal")
    finally:
        c.close()


def test_route_without_renormalization(cx):
    P, pr = cx.P, cx.pr
    E, top_k, hidden, rows = 8, 2, 256, 5
    router = o.normal(11, 0.02, E * hidden).reshape(E, hidden)
    x = o.normal(12, 1.0, rows * hidden).reshape(rows, hidden)
    key = {"op": {"MoeRoute": {"norm": "Softmax"}}, "schemes": [{"Plain": "F32"}, {"Plain": "F32"}],
           "layout": 0, "variant": 0}
    announce("provider route renormalize=0")
    op = pr.prepare(cx.ctx, key, shape(rows, E, top_k, hidden))
    rd = dev(router)
    xb, ids_b, w_b = cx.put(x), cx.empty(4 * rows * top_k), cx.empty(4 * rows * top_k)
    pr.launch(cx.ctx, cx.s, op, P.op_args([P.packed(xb, P.DT_F32, [rows, hidden])],
                                          [P.packed(ids_b, P.DT_I32, [rows, top_k]),
                                           P.packed(w_b, P.DT_F32, [rows, top_k])],
                                          [P.view(rd.data_ptr(), router.nbytes)], cx.workspace(op),
                                          [P.Scalar(2, 0)]))
    wids, ww, _ = o.moe_route(router, x, E, top_k, False)
    assert (cx.get(ids_b, np.int32, (rows, top_k)) == wids).all()
    assert_same(cx.get(w_b, np.float32, (rows, top_k)), ww)


def test_capture_and_replay(cx):
    """A captured Q4_K GEMV replayed three times over new inputs written between replays; every
    replay equals the oracle."""
    P, pr = cx.P, cx.pr
    rows, n_out, k = 4, 768, 2048
    rng = GemvRng(4242)
    w = gemv_weights(rng, o.Q4_K, n_out, k, o.f16_bits, o.round_bf16)
    op = pr.prepare(cx.ctx, gemv_key(o.Q4_K), shape(rows, n_out, k))
    wd = dev(w)
    xb, yb = cx.empty(4 * rows * k, 0), cx.empty(4 * rows * n_out)
    args = P.op_args([P.packed(xb, P.DT_F32, [rows, k])], [P.packed(yb, P.DT_F32, [rows, n_out])],
                     [P.view(wd.data_ptr(), w.nbytes)], cx.workspace(op))
    announce("provider capture/replay")
    pr.begin_capture(cx.ctx, cx.s)
    pr.launch(cx.ctx, cx.s, op, args)
    g = pr.end_capture(cx.ctx, cx.s)
    for i in range(3):
        x = gemv_activations(rng, rows, k).astype(np.float32)
        cx.upload(xb.addr, x)
        pr.replay(cx.ctx, cx.s, g)
        got = cx.get(yb, np.float32, (rows, n_out))
        assert_same(got, o.gemv(o.Q4_K, w, n_out, k, x, rows, threads=8), f"replay {i}")


def test_events_and_device_copy(cx):
    P, pr = cx.P, cx.pr
    a = np.arange(1 << 16, dtype=np.uint32)
    src, dst = cx.put(a), cx.empty(a.nbytes, 0)
    e0, e1 = pr.event(cx.ctx), pr.event(cx.ctx)
    announce("provider copy + events")
    pr.record(cx.ctx, cx.s, e0)
    pr.copy(cx.ctx, cx.s, P.Slice(src.handle, 0, a.nbytes), P.Slice(dst.handle, 0, a.nbytes))
    pr.record(cx.ctx, cx.s, e1)
    assert (cx.get(dst, np.uint32, a.size) == a).all()
    assert pr.poll(cx.ctx, e1)
    mi = pr.memory_info(cx.ctx)
    assert mi.total > 200 << 30 and 0 < mi.free <= mi.total
    devs = pr.enumerate()
    assert devs and devs[0]["class"] == {"Hip": {"gfx": 0x950}}
    with pytest.raises(P.ProviderError):  # a slice past its buffer
        pr.copy(cx.ctx, cx.s, P.Slice(src.handle, 8, a.nbytes), P.Slice(dst.handle, 0, a.nbytes))
