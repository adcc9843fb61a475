"""The provider-library boundary on the CPU: the one exported symbol, the header handshake, the
table's identity and layout, the JSON the core reads (ops, query), and the error protocol
(status classes and codes, per-thread messages, per-thread contexts, stickiness).  No device call
reaches a kernel: on a host without a GPU `open` fails with a Device status.

The reference's own checks of a module: crates/kernels-loader/src/module.rs:26-40 (header),
crates/kernels/src/abi/guest.rs:184-280 (status, messages, contexts)."""
import ctypes as C
import json
import os
import subprocess
import sys
import threading

import pytest

import torch  # noqa: F401  one HIP runtime in the process

from syntropy_amd import provider as P

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def pr():
    if not os.path.exists(P.PROVIDER_LIB):
        pytest.fail(f"{P.PROVIDER_LIB} is not built: run python -m syntropy_amd.build")
    return P.Provider()


def test_the_dynamic_symbol_table_holds_exactly_the_entry_symbol():
    """crates/kernels-loader/tests/exports.rs:48-70: `nm -D --defined-only` lists the entry symbol
    and nothing else (the version node, when the linker lists it, is an absolute symbol); the
    entry is under the version node SYNTROPY_PROVIDER_1."""
    out = subprocess.run(["nm", "-D", "--defined-only", P.PROVIDER_LIB], capture_output=True, text=True,
                         check=True).stdout
    lines = [l for l in out.splitlines() if l.split() and not l.rstrip().endswith("A SYNTROPY_PROVIDER_1")]
    names = [l.split()[-1] for l in lines]
    assert [n.split("@")[0] for n in names] == ["syntropy_provider_entry_v1"], out
    assert names[0].endswith("@@SYNTROPY_PROVIDER_1"), out


STICKY_SCRIPT = r"""
import json, sys
import torch  # one HIP runtime in the process
from syntropy_amd import provider as P
P.CONFIG.update(json.loads(sys.argv[1]))
pr = P.Provider()
res = {}
def run(name, f):
    st = f()
    res[name] = [st.cls, st.code, st.domain, pr.message()]
run("ops", lambda: pr.vt.ops(pr.vt.slf, P.OutBuf()))
run("build", lambda: pr.vt.build(pr.vt.slf, P.OutBuf()))
h = P.Health()
run("health", lambda: pr.vt.health(pr.vt.slf, 0, h))
res["health_state"] = [h.kind, h.domain, h.detail]
res["log"] = P.LOG
print(json.dumps(res))
"""


def sticky_run(config):
    r = subprocess.run([sys.executable, "-c", STICKY_SCRIPT, json.dumps(config)], capture_output=True, text=True,
                       cwd=ROOT, timeout=300)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_a_caught_panic_makes_the_provider_sticky():
    """fixture.panic_in names an entry that throws (the reference's test provider key,
    crates/kernels-loader/examples/test_provider.rs:7-16): that call returns Internal /
    ProviderPanicked (16); every later entry but health, free and close_ctx returns Device /
    DeviceSticky (8); health reports Sticky (kind 3) with code 16; the host's log has the error
    (crates/kernels/src/abi/guest.rs:184-230)."""
    r = sticky_run({"fixture.panic_in": "ops"})
    assert r["ops"][:3] == [P.CLASS_INTERNAL, P.CODE_PROVIDER_PANICKED, 1]
    assert "injected by fixture.panic_in" in r["ops"][3]
    assert r["build"][:3] == [P.CLASS_DEVICE, P.CODE_DEVICE_STICKY, 1]
    assert "sticky after code 16" in r["build"][3]
    assert r["health"][0] == 0 and r["health_state"] == [3, 1, 16]
    assert any(level == 0 and "injected by fixture.panic_in" in msg for level, _, msg in r["log"])


def test_a_sticky_device_error_makes_the_provider_sticky():
    """fixture.device_fault_in makes an entry meet an illegal-address error, as a faulted kernel
    reports it: Device / DeviceSticky (8), the provider sticky with that code (RFC-0040 ...md:861,
    933)."""
    r = sticky_run({"fixture.device_fault_in": "build"})
    assert r["ops"][0] == 0
    assert r["build"][:3] == [P.CLASS_DEVICE, P.CODE_DEVICE_STICKY, 1]
    assert "the provider is sticky" in r["build"][3]
    assert r["health_state"] == [3, 1, 8]
    assert any(level == 0 and "fixture.device_fault_in" in msg for level, _, msg in r["log"])


def test_no_injection_leaves_the_provider_healthy():
    r = sticky_run({})
    assert r["ops"][0] == 0 and r["build"][0] == 0 and r["health_state"] == [0, 0, 0] and r["log"] == []


def test_struct_sizes_match_the_reference_layout():
    # repr(C) sizes of crates/kernels/src/abi/types.rs on x86-64
    assert C.sizeof(P.Header) == 52
    assert C.sizeof(P.Status) == 12
    assert C.sizeof(P.TensorArg) == 64
    assert C.sizeof(P.BufferView) == 56
    assert C.sizeof(P.OpArgs) == 120
    assert C.sizeof(P.Health) == P.HEALTH_SIZE
    assert C.sizeof(P.Vtbl) == 24 + 36 * 8 + 8 + 8  # head, 36 entries, slf, health_size (padded)


def test_python_mirror_matches_the_c_header(tmp_path):
    """Every field offset of the ctypes mirror equals the C header's (compiled here with gcc)."""
    pairs = [("SynHeader", P.Header), ("SynStatus", P.Status), ("SynHostApi", P.HostApi),
             ("SynMemoryInfo", P.MemoryInfo), ("SynBuffer", P.Buffer), ("SynSlice", P.Slice),
             ("SynTensorArg", P.TensorArg), ("SynBufferView", P.BufferView), ("SynOpArgs", P.OpArgs),
             ("SynOutBuf", P.OutBuf), ("SynProviderVtbl", P.Vtbl), ("SynModule", P.Module),
             ("SynOpenOptions", P.OpenOptions), ("SynDeviceId", P.DeviceId)]
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "syntropy_provider.h"', "int main(void){"]
    want = []
    for cname, py in pairs:
        lines.append(f'printf("%zu\\n", sizeof({cname}));')
        want.append(C.sizeof(py))
        for f, _ in py._fields_:
            lines.append(f'printf("%zu\\n", offsetof({cname}, {f}));')
            want.append(getattr(py, f).offset)
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == want


def test_refuses_a_foreign_host_header():
    for kw in ({"magic": b"SYNPROV2"}, {"major": 2}, {"size": 16}):
        m, _, _ = P.load(host=P.host_api(**kw))
        assert m is None, kw
    m, _, _ = P.load()
    assert m is not None and bytes(m.h.magic) == P.MAGIC


def test_module_and_table_identity(pr):
    m, vt = pr.module, pr.vt
    assert (m.h.abi_major, m.h.abi_minor, m.n_providers) == (1, 0, 1)
    assert m.h.struct_size == C.sizeof(P.Module)
    assert vt.struct_size == C.sizeof(P.Vtbl)
    assert pr.id() == "hip" and vt.backend == P.BACKEND_HIP and vt.domain == P.MEMDOMAIN_HIP
    assert vt.health_size == 12
    assert m.shutdown().cls == 0


def test_build_and_ops_json(pr):
    b = pr.build()
    assert b["version"] == 1 and ["target", "gfx950"] in b["toolchain"]
    ops = pr.ops()
    got = {(json.dumps(k["op"]), json.dumps(k["schemes"][0]), k["layout"]) for k in ops}
    weights = [('{"Ggml": "Q4_K"}', 0), ('{"Ggml": "Q4_K"}', 1), ('{"Ggml": "Q8_0"}', 0), ('{"Ggml": "Q4_0"}', 0),
               ('{"Ggml": "Q8_0"}', 2), ('{"Ggml": "Q4_0"}', 2),
               ('{"Ggml": "F16"}', 0), ('{"Ggml": "BF16"}', 0), ('{"Plain": "F16"}', 0), ('{"Plain": "BF16"}', 0)]
    dense = {(op, w, l) for op in ('"Gemv"', '"Gemm"', '"Logits"', '{"GateUpAct": {"act": "Silu"}}')
             for w, l in weights}
    assert got == dense | {('"MoeGrouped"', '{"Ggml": "Q4_K"}', 0), ('"MoeGrouped"', '{"Ggml": "Q8_0"}', 0),
                           ('{"MoeRoute": {"norm": "Softmax"}}', '{"Plain": "F32"}', 0),
                           ('"MoeCombine"', '{"Plain": "F32"}', 0)}
    assert len(ops) == len(got)
    for k in ops:
        assert k["variant"] == 0


def test_outbuf_retry_protocol(pr):
    """A too-small buffer gets only the length (types.rs SynOutBuf)."""
    buf = (C.c_uint8 * 4)(9, 9, 9, 9)
    out = P.OutBuf(C.cast(buf, C.POINTER(C.c_uint8)), 4, 0)
    assert pr.vt.ops(pr.vt.slf, C.byref(out)).cls == 0
    assert out.len > 4 and list(buf) == [9, 9, 9, 9]


def test_unserved_entries_are_unsupported(pr):
    vt, slf = pr.vt, pr.vt.slf
    calls = {
        "map_segment": lambda: vt.map_segment(slf, 1, None, 0, 0, None),
        "unmap_segment": lambda: vt.unmap_segment(slf, 1, None),
        "register_host": lambda: vt.register_host(slf, 1, P.HostRegion(0, 0), None),
        "host_registrar": lambda: vt.host_registrar(slf, 1, None),
        "import": lambda: getattr(vt, "import")(slf, 1, P.HostRegion(0, 0), None),
        "arm_wake": lambda: vt.arm_wake(slf, 1, 1, 3, 0),  # TimelineValue: not served
    }
    for name, f in calls.items():
        st = f()
        assert (st.cls, st.code, st.domain) == (2, 1, 1), name
        assert name in pr.message(), name


def test_arm_wake_serves_futex_and_eventfd_only(pr):
    """WakeKind codes (crates/kernels/src/abi/wire.rs:180-197): Futex 0 and EventFd 1 are
    served (checked against the context next), WinEvent 2 and TimelineValue 3 are Unsupported."""
    vt, slf = pr.vt, pr.vt.slf
    for kind in (2, 3):
        st = vt.arm_wake(slf, 987654, 1, kind, 5)
        assert (st.cls, st.code) == (2, 1), kind
    for kind in (0, 1):
        assert vt.arm_wake(slf, 987654, 1, kind, 64).cls == 13, kind


def test_doorbell_entries_check_their_context(pr):
    """signal_host and wait_host are served; on a context not open on this thread they refuse
    with Internal before anything is enqueued (the CPU provider's flag_slot check,
    crates/kernels-cpu/src/provider.rs:187-192, comes after its context check)."""
    vt, slf = pr.vt, pr.vt.slf
    for name, st in [("signal_host", vt.signal_host(slf, 987654, 1, 0, 1)),
                     ("wait_host", vt.wait_host(slf, 987654, 1, 0, 1, 0, 1, 0))]:
        assert st.cls == 13, name
        assert "not open on this thread" in pr.message(), name


def _key(op, weight, layout=0):
    schemes = ([{"Ggml": weight}] if weight else []) + [{"Plain": "F32"}, {"Plain": "F32"}]
    return json.dumps({"op": op, "schemes": schemes, "layout": layout, "variant": 0}).encode()


def test_repack_of_q4k_gemv_is_the_x8_permutation(pr):
    """Gemv's Q4_K weights repack to layout 1 (each run of eight super-blocks chunk-major, the
    same length); every other op keeps the source layout (provider.rs:326-336)."""
    import numpy as np
    nblk = 21
    src = np.random.default_rng(1).integers(0, 256, nblk * 144, dtype=np.uint8)
    want = np.empty_like(src)
    for g0 in range(0, nblk, 8):
        m = min(8, nblk - g0)
        want[g0 * 144:(g0 + m) * 144] = src[g0 * 144:(g0 + m) * 144].reshape(m, 9, 16).transpose(1, 0, 2).ravel()
    present, layout, n = C.c_uint32(7), C.c_uint32(7), C.c_uint64(7)
    key = _key("Gemv", "Q4_K")
    kb = (C.c_uint8 * len(key)).from_buffer_copy(key)
    assert pr.vt.repacked_len(pr.vt.slf, kb, len(key), src.size, C.byref(present), C.byref(n)).cls == 0
    assert (present.value, n.value) == (1, src.size)
    dst = np.zeros_like(src)
    sp, dp = src.ctypes.data_as(C.POINTER(C.c_uint8)), dst.ctypes.data_as(C.POINTER(C.c_uint8))
    assert pr.vt.repack(pr.vt.slf, kb, len(key), sp, src.size, dp, dst.size, C.byref(present), C.byref(layout)).cls == 0
    assert (present.value, layout.value) == (1, 1)
    assert (dst == want).all()
    for dense_op in ("Gemm", "Logits", {"GateUpAct": {"act": "Silu"}}):
        kd = _key(dense_op, "Q4_K")
        db = (C.c_uint8 * len(kd)).from_buffer_copy(kd)
        assert pr.vt.repacked_len(pr.vt.slf, db, len(kd), src.size, C.byref(present), C.byref(n)).cls == 0
        assert (present.value, n.value) == (1, src.size)
    for other in (_key("Gemv", "F16"), _key("MoeGrouped", "Q4_K"), _key("MoeGrouped", "Q8_0"),
                  _key("MoeCombine", None)):
        ob = (C.c_uint8 * len(other)).from_buffer_copy(other)
        assert pr.vt.repacked_len(pr.vt.slf, ob, len(other), 144, C.byref(present), C.byref(n)).cls == 0
        assert (present.value, n.value) == (0, 0)
        assert pr.vt.repack(pr.vt.slf, ob, len(other), sp, 144, dp, 144, C.byref(present), C.byref(layout)).cls == 0
        assert (present.value, layout.value) == (0, 0)
    bad = pr.vt.repack(pr.vt.slf, kb, len(key), sp, 100, dp, 100, C.byref(present), C.byref(layout))
    assert bad.cls == 1 and "super-blocks" in pr.message()


@pytest.mark.parametrize("wname,bb", [("Q8_0", 34), ("Q4_0", 18)])
def test_repack_of_q8_0_and_q4_0_dense_weights_is_the_split_layout(pr, wname, bb):
    """The dense products' Q8_0 and Q4_0 weights repack to layout 2 (every block's codes, then
    every block's F16 scale, the same length)."""
    import numpy as np
    nblk = 37
    src = np.random.default_rng(bb).integers(0, 256, nblk * bb, dtype=np.uint8)
    blocks = src.reshape(nblk, bb)
    want = np.concatenate([blocks[:, 2:].ravel(), blocks[:, :2].ravel()])
    present, layout, n = C.c_uint32(7), C.c_uint32(7), C.c_uint64(7)
    sp = src.ctypes.data_as(C.POINTER(C.c_uint8))
    for op in ("Gemv", "Gemm", "Logits", {"GateUpAct": {"act": "Silu"}}):
        key = _key(op, wname)
        kb = (C.c_uint8 * len(key)).from_buffer_copy(key)
        assert pr.vt.repacked_len(pr.vt.slf, kb, len(key), src.size, C.byref(present), C.byref(n)).cls == 0
        assert (present.value, n.value) == (1, src.size)
        dst = np.zeros_like(src)
        dp = dst.ctypes.data_as(C.POINTER(C.c_uint8))
        assert pr.vt.repack(pr.vt.slf, kb, len(key), sp, src.size, dp, dst.size, C.byref(present),
                            C.byref(layout)).cls == 0
        assert (present.value, layout.value) == (1, 2)
        assert (dst == want).all()
    bad = pr.vt.repack(pr.vt.slf, kb, len(key), sp, src.size - 1, dp, dst.size, C.byref(present), C.byref(layout))
    assert bad.cls == 1 and "32-value blocks" in pr.message()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour on a host without a GPU")
def test_open_without_a_device_is_a_device_error(pr):
    with pytest.raises(P.ProviderError) as e:
        pr.open(0)
    assert e.value.cls == 6 and "no HIP device" in e.value.message
    assert pr.enumerate() == []


def test_unknown_context_is_refused(pr):
    with pytest.raises(P.ProviderError) as e:
        pr.query(987654, {"op": "Gemv"}, {})
    assert e.value.cls == 13 and "not open on this thread" in e.value.message
    with pytest.raises(P.ProviderError):
        pr.stream(987654)
    with pytest.raises(P.ProviderError):
        pr.close(987654)


def test_messages_are_per_thread(pr):
    with pytest.raises(P.ProviderError):
        pr.stream(5551)
    mine = pr.message()
    seen = {}

    def other():
        seen["before"] = pr.message()
        st = pr.vt.map_segment(pr.vt.slf, 1, None, 0, 0, None)
        seen["cls"] = st.cls
        seen["after"] = pr.message()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "5551" in mine
    assert seen["before"] == "" and seen["cls"] == 2 and "map_segment" in seen["after"]
    assert pr.message() == mine


def test_health_is_healthy(pr):
    h = pr.health()
    assert (h.kind, h.domain, h.detail) == (0, 0, 0)


def test_header_declares_the_entry():
    text = open(os.path.join(ROOT, "include", "syntropy_provider.h")).read()
    assert "const SynModule* syntropy_provider_entry_v1(const SynHostApi* host);" in text
