"""The C-ABI library loads and exports every function its public headers declare.

CPU-only: loads the shared object and resolves symbols; makes no compute calls.
"""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "syntropy_amd", "libsyntropy_hip.so")
PROVIDER_LIB = os.path.join(ROOT, "syntropy_amd", "libsyntropy_provider.so")
# which library exports what each header declares
HEADER_LIB = {"syntropy_hip.h": LIB, "syntropy_provider.h": PROVIDER_LIB}


def declared_functions(header=None):
    names = []
    for h in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))):
        if header is not None and os.path.basename(h) != header:
            continue
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*(?:\s+\**|\s*\*+)\s*\**\s*([a-z][a-z0-9_]*)\s*\(",
                             text, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))


def test_headers_declare_functions():
    names = declared_functions()
    assert "syn_gemv" in names and "syn_last_error" in names


def test_every_header_has_its_library():
    headers = sorted(os.path.basename(h) for h in glob.glob(os.path.join(ROOT, "include", "*.h")))
    assert headers == sorted(HEADER_LIB)


@pytest.mark.parametrize("header", sorted(HEADER_LIB))
def test_library_exports_every_declared_function(header):
    path = HEADER_LIB[header]
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built: run python -m syntropy_amd.build")
    import torch  # noqa: F401  one HIP runtime in the process
    lib = ctypes.CDLL(path)
    names = declared_functions(header)
    assert names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_errors_without_a_gpu():
    import torch  # noqa: F401
    lib = ctypes.CDLL(LIB)
    lib.syn_version.restype = ctypes.c_int
    assert lib.syn_version() >= 100
    lib.syn_last_error.restype = ctypes.c_char_p
    out = ctypes.c_uint64()
    # a refused call (Q4_K rows of 100 values) reports through syn_last_error, touching no device
    lib.syn_gemv_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.POINTER(ctypes.c_uint64)]
    assert lib.syn_gemv_workspace_bytes(12, 1, 100, ctypes.byref(out)) == 1
    assert b"256" in lib.syn_last_error()
    assert lib.syn_gemv_workspace_bytes(12, 1, 4096, ctypes.byref(out)) == 0
    assert out.value >= 4096 + 16 * 4 + 128 * 4
    assert lib.syn_gemv_workspace_bytes(7, 1, 4096, ctypes.byref(out)) == 2


def test_x8_host_repack_is_its_definition_and_inverts():
    """The host repack of the X8 layout against its definition (chunk q of block i of a run of m
    at 16 (q m + i)), and the inverse; no device involved."""
    import numpy as np
    import torch  # noqa: F401
    lib = ctypes.CDLL(LIB)
    lib.syn_q4k_repack_host.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                        ctypes.c_int32]
    for nblk in (1, 7, 8, 9, 21, 64):
        b = np.random.default_rng(nblk).integers(0, 256, nblk * 144, dtype=np.uint8)
        want = np.empty_like(b)
        for g0 in range(0, nblk, 8):
            m = min(8, nblk - g0)
            want[g0 * 144:(g0 + m) * 144] = b[g0 * 144:(g0 + m) * 144].reshape(m, 9, 16).transpose(1, 0, 2).ravel()
        got = np.empty_like(b)
        assert lib.syn_q4k_repack_host(1, b.ctypes.data, got.ctypes.data, b.size, 0) == 0
        assert (got == want).all()
        back = np.empty_like(b)
        assert lib.syn_q4k_repack_host(1, got.ctypes.data, back.ctypes.data, b.size, 1) == 0
        assert (back == b).all()
    assert lib.syn_q4k_repack_host(2, b.ctypes.data, got.ctypes.data, b.size, 0) == 2
    assert lib.syn_q4k_repack_host(1, b.ctypes.data, got.ctypes.data, 100, 0) == 1


def test_split_host_repack_is_its_definition_and_inverts():
    """The host repack of the SPLIT layout (every block's codes, then every block's F16 scale)
    against its definition, and the inverse, for Q8_0 (34-byte blocks) and Q4_0 (18)."""
    import numpy as np
    import torch  # noqa: F401
    lib = ctypes.CDLL(LIB)
    lib.syn_split_repack_host.argtypes = [ctypes.c_uint32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_uint64, ctypes.c_int32]
    for ty, bb in ((8, 34), (2, 18)):
        for nblk in (1, 7, 64, 129):
            b = np.random.default_rng(nblk + ty).integers(0, 256, nblk * bb, dtype=np.uint8)
            blocks = b.reshape(nblk, bb)
            want = np.concatenate([blocks[:, 2:].ravel(), blocks[:, :2].ravel()])
            got = np.empty_like(b)
            assert lib.syn_split_repack_host(2, ty, b.ctypes.data, got.ctypes.data, b.size, 0) == 0
            assert (got == want).all()
            back = np.empty_like(b)
            assert lib.syn_split_repack_host(2, ty, got.ctypes.data, back.ctypes.data, b.size, 1) == 0
            assert (back == b).all()
        assert lib.syn_split_repack_host(1, ty, b.ctypes.data, got.ctypes.data, b.size, 0) == 2
        assert lib.syn_split_repack_host(2, ty, b.ctypes.data, got.ctypes.data, b.size - 1, 0) == 1
    assert lib.syn_split_repack_host(2, 12, b.ctypes.data, got.ctypes.data, 144, 0) == 2


def test_tile64_host_repack_is_its_definition_and_inverts():
    """The host repack of the TILE64 layout (within each run of 64 rows, super-block b of row r at
    144 (64 b + r)) against an element-wise placement loop, and the inverse; stacks of one and
    three runs, rows of 1, 6 and 16 super-blocks; lengths that are not whole runs are refused."""
    import numpy as np
    import torch  # noqa: F401
    lib = ctypes.CDLL(LIB)
    lib.syn_q4k_tile64_repack_host.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                               ctypes.c_uint32, ctypes.c_int32]
    for nb, runs in ((1, 1), (6, 3), (16, 2)):
        rows, rb = 64 * runs, nb * 144
        b = np.random.default_rng(nb * 10 + runs).integers(0, 256, rows * rb, dtype=np.uint8)
        want = np.empty_like(b)
        for r in range(rows):
            for j in range(nb):
                at = (r // 64) * 64 * rb + 144 * (64 * j + r % 64)
                want[at:at + 144] = b[r * rb + 144 * j:r * rb + 144 * (j + 1)]
        got = np.empty_like(b)
        assert lib.syn_q4k_tile64_repack_host(b.ctypes.data, got.ctypes.data, b.size, 256 * nb, 0) == 0
        assert (got == want).all()
        back = np.empty_like(b)
        assert lib.syn_q4k_tile64_repack_host(got.ctypes.data, back.ctypes.data, b.size, 256 * nb, 1) == 0
        assert (back == b).all()
    assert lib.syn_q4k_tile64_repack_host(b.ctypes.data, got.ctypes.data, b.size - rb, 256 * nb, 0) == 1
    assert lib.syn_q4k_tile64_repack_host(b.ctypes.data, got.ctypes.data, b.size, 300, 0) == 1
