"""syn_gemv_layout_noalloc (the Gemv whose workspace is the library's per-device scratch array)
against syn_gemv_layout with a caller workspace, through the C ABI: bit-identical outputs on two
calls in a row, the second on a smaller input, so leftovers of the first call in the shared
array must not reach the second; and the oracle's values."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import announce, assert_same, dev, host, require_gpu
from oracle import oracle as o
from test_gpu_gemm import random_q4k

pytestmark = pytest.mark.gpu

SOURCE, X8 = 0, 1


@pytest.fixture(scope="module")
def L():
    require_gpu()
    from syntropy_amd import _lib
    lib = _lib.lib()
    vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32
    lib.syn_gemv_layout_noalloc.argtypes = [u32, i32, vp, u64, u32, u32, vp, u32, vp, vp]
    lib.syn_gemv_layout_noalloc.restype = C.c_int
    lib.syn_gemv_layout_noalloc_max_workspace.argtypes = []
    lib.syn_gemv_layout_noalloc_max_workspace.restype = u64
    return lib


def weights(L, layout, ty, n_out, k, seed):
    rs = np.random.default_rng(seed)
    if ty == o.Q4_K:
        w = random_q4k(rs, n_out, k)
    else:
        w = o.quantize(ty, o.normal(seed, 0.02, n_out * k))
    wd = dev(w)
    if layout == X8:
        r = torch.empty_like(wd)
        assert L.syn_q4k_repack(X8, wd.data_ptr(), r.data_ptr(), wd.numel(), 0, None) == 0
        wd = r
    return w, wd


def with_workspace(L, layout, ty, wd, n_out, k, xd, rows):
    need = C.c_uint64(0)
    assert L.syn_gemv_layout_workspace_bytes(layout, ty, rows, k, C.byref(need)) == 0
    ws = torch.full((need.value + 256,), 0xA5, dtype=torch.uint8, device="cuda")
    base = (ws.data_ptr() + 255) // 256 * 256
    y = torch.full((rows, n_out), float("nan"), device="cuda")
    rc = L.syn_gemv_layout(layout, ty, wd.data_ptr(), wd.numel(), n_out, k, xd.data_ptr(), rows,
                           y.data_ptr(), base, need.value, None)
    assert rc == 0, L.syn_last_error().decode()
    return host(y)


def no_alloc(L, layout, ty, wd, n_out, k, xd, rows):
    y = torch.full((rows, n_out), float("nan"), device="cuda")
    rc = L.syn_gemv_layout_noalloc(layout, ty, wd.data_ptr(), wd.numel(), n_out, k, xd.data_ptr(),
                                   rows, y.data_ptr(), None)
    assert rc == 0, L.syn_last_error().decode()
    return host(y)


# (layout, weight type, n_out, k, rows): each pair is a larger call then a smaller one
CASES = [
    [(X8, o.Q4_K, 1024, 14336, 64), (X8, o.Q4_K, 300, 4096, 40)],   # the matrix-core GEMM
    [(X8, o.Q4_K, 4096, 14336, 1), (X8, o.Q4_K, 4096, 4096, 1)],    # the decode kernel
    [(SOURCE, o.Q8_0, 2048, 4096, 8), (SOURCE, o.Q8_0, 512, 1024, 3)],
    [(SOURCE, o.Q4_K, 512, 4096, 33), (SOURCE, o.Q4_0, 256, 2048, 2)],
]


@pytest.mark.parametrize("pair", CASES, ids=lambda p: "-".join(f"{c[0]}:{c[1]}:{c[2]}x{c[3]}r{c[4]}" for c in p))
def test_no_alloc_equals_the_workspace_entry(L, pair):
    for i, (layout, ty, n_out, k, rows) in enumerate(pair):
        w, wd = weights(L, layout, ty, n_out, k, 0x70 + i + n_out)
        x = o.normal(0x71 + rows + k, 1.0, rows * k).reshape(rows, k)
        xd = dev(x)
        announce(f"no-alloc call {i}: layout {layout} type {ty} {n_out}x{k} rows {rows}")
        want = with_workspace(L, layout, ty, wd, n_out, k, xd, rows)
        got = no_alloc(L, layout, ty, wd, n_out, k, xd, rows)
        assert_same(got, want, f"call {i} vs the workspace entry")
        assert_same(got, o.gemv(ty, w, n_out, k, x, rows, threads=16), f"call {i} vs the oracle")


def test_no_alloc_refuses_workspaces_beyond_the_scratch(L):
    cap = L.syn_gemv_layout_noalloc_max_workspace()
    assert cap == 8 << 20
    rows, k = 2048, 4096  # 2048 x 4096 activations in the GEMM layout: above 8 MiB
    need = C.c_uint64(0)
    assert L.syn_gemv_layout_workspace_bytes(X8, o.Q4_K, rows, k, C.byref(need)) == 0
    assert need.value > cap
    y = torch.empty(rows, 64, device="cuda")
    x = torch.zeros(rows, k, device="cuda")
    w = torch.zeros(64 * (k // 256) * 144, dtype=torch.uint8, device="cuda")
    rc = L.syn_gemv_layout_noalloc(X8, o.Q4_K, w.data_ptr(), w.numel(), 64, k, x.data_ptr(), rows,
                                   y.data_ptr(), None)
    assert rc == 2, rc  # SYN_E_UNSUPPORTED
    assert "scratch" in L.syn_last_error().decode()
