"""Helpers of the GPU tests: device transfer, bit comparison, and the library under test."""
from __future__ import annotations

import sys

import numpy as np
import torch


def require_gpu():
    """GPU tests fail, never skip, on a host without the device (they are selected by -m gpu)."""
    assert torch.cuda.is_available(), "this test needs an MI355X"
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert "gfx950" in name, f"expected gfx950, found {name}"


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def assert_same(got, want, what=""):
    """Bit-equal, or both NaN (crates/kernels-cpu/src/gemv/tests.rs:147-162)."""
    got = np.asarray(got, dtype=np.float32).ravel()
    want = np.asarray(want, dtype=np.float32).ravel()
    assert got.shape == want.shape, f"{what}: shapes {got.shape} {want.shape}"
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    if not same.all():
        i = int(np.flatnonzero(~same)[0])
        raise AssertionError(f"{what}: {int((~same).sum())} of {got.size} differ; first at {i}: "
                             f"{got[i]!r} ({bits(got)[i]:#010x}) != {want[i]!r} ({bits(want)[i]:#010x})")


def announce(msg: str):
    """Names the case on stdout before a GPU step, so a fault still tells which case ran."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()
