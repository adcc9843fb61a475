"""Loads libsyntropy_hip.so (the C ABI of include/syntropy_hip.h) with ctypes.

The library must share the process's HIP runtime with PyTorch, so torch is imported first:
both then bind the one libamdhip64.so.7 already loaded.  A missing library is an error, never a
silent fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsyntropy_hip.so")

_lib = None


class SynError(RuntimeError):
    """A refused or failed call; `code` is the SYN_E_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (one HIP runtime for torch and the library)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m syntropy_amd.build` "
            "(the HIP path has no fallback)")
    L = C.CDLL(LIB_PATH)
    vp, i32, u32, u64, fp = C.c_void_p, C.c_int32, C.c_uint32, C.c_uint64, C.c_void_p
    L.syn_last_error.restype = C.c_char_p
    L.syn_version.restype = C.c_int
    sigs = {
        "syn_gemv_workspace_bytes": [i32, u32, u32, C.POINTER(C.c_uint64)],
        "syn_act_quantize": [i32, fp, u32, u32, vp, u64, vp],
        "syn_gemv_quantized": [i32, vp, u64, u32, u32, vp, u64, u32, fp, vp],
        "syn_gemv": [i32, vp, u64, u32, u32, fp, u32, fp, vp, u64, vp],
        "syn_quantize": [i32, fp, u64, vp, u64, vp],
        "syn_gemv_batch_workspace_bytes": [u32, vp, C.POINTER(C.c_uint64)],
        "syn_gemv_batch": [u32, vp, vp, vp, vp, vp, vp, vp, vp, u64, vp],
        "syn_act_quantize_batch": [u32, vp, vp, vp, u64, vp],
        "syn_gemv_batch_quantized": [u32, vp, vp, vp, vp, vp, vp, u64, vp, vp],
        "syn_dequantize": [i32, vp, u64, fp, vp],
        "syn_gemm_workspace_bytes": [u32, u32, C.POINTER(C.c_uint64)],
        "syn_gemm_act_quantize": [vp, u32, u32, vp, u64, vp],
        "syn_gemm_q4k_quantized": [vp, u64, u32, u32, vp, u64, u32, vp, vp],
        "syn_q4k_repack": [u32, vp, vp, u64, i32, vp],
        "syn_q4k_repack_host": [u32, vp, vp, u64, i32],
        "syn_split_repack": [u32, i32, vp, vp, u64, i32, vp],
        "syn_gemv_quantized_layout": [u32, i32, vp, u64, u32, u32, vp, u64, u32, vp, vp],
        "syn_split_repack_host": [u32, i32, vp, vp, u64, i32],
        "syn_gemv_layout_workspace_bytes": [u32, i32, u32, u32, C.POINTER(C.c_uint64)],
        "syn_gemv_layout": [u32, i32, vp, u64, u32, u32, vp, u32, vp, vp, u64, vp],
        "syn_gate_up_act_workspace_bytes": [u32, i32, u32, u32, u32, vp],
        "syn_gate_up_act": [u32, i32, vp, u64, u32, u32, vp, u32, vp, vp, u64, vp],
        "syn_gemv_batch_layout": [u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, u64, vp],
        "syn_gemv_batch_quantized_layout": [u32, u32, vp, vp, vp, vp, vp, vp, u64, vp, vp],
        "syn_hbm_read_probe": [vp, u64, vp, vp],
        "syn_hbm_read_runs": [u32, vp, u64, vp, vp],
        "syn_div_forms_check": [vp, vp],
        "syn_rms_norm": [vp, vp, u32, u32, C.c_float, vp, vp],
        "syn_logits_workspace_bytes": [u32, i32, u32, u32, u32, C.POINTER(C.c_uint64)],
        "syn_logits": [u32, i32, vp, u64, u32, u32, vp, C.c_float, vp, u32, vp, vp, u64, vp],
        "syn_moe_route": [vp, vp, u32, u32, u32, u32, i32, vp, vp, vp, vp],
        "syn_moe_pack": [vp, u32, u32, u32, vp, vp, vp, vp],
        "syn_moe_grouped_workspace_bytes": [i32, u32, u32, u32, u32, u32, C.POINTER(C.c_uint64)],
        "syn_moe_grouped": [i32, vp, vp, vp, u64, u32, u32, u32, u32, vp, vp, vp, u32, vp, vp, u64, vp, vp],
        "syn_moe_grouped_layout": [u32, i32, vp, vp, vp, u64, u32, u32, u32, u32, vp, vp, vp, u32, vp, vp, u64, vp,
                                   vp],
        "syn_q4k_tile64_repack": [vp, vp, u64, u32, i32, vp],
        "syn_q4k_tile64_repack_host": [vp, vp, u64, u32, i32],
        "syn_moe_doorbell": [vp, u32, u32, u32, vp, vp, u32, vp, u32, vp, vp],
        "syn_moe_assign": [vp, u32, vp, u32, u32, u64, u32, vp, vp],
        "syn_moe_assign_layer": [vp, u32, vp, u32, vp, u64, u32, vp, vp],
        "syn_moe_site_mask": [vp, u32, vp, u32, i32, vp, vp],
        "syn_moe_combine": [vp, vp, vp, u32, u32, u32, vp, vp],
        "syn_moe_combine_ranked": [vp, vp, u32, vp, u32, u32, u32, vp, vp],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = C.c_int
    _lib = L
    return L


def bind(name: str, argtypes, restype=C.c_int):
    """Declares one more C entry point (used by modules that add functions)."""
    f = getattr(lib(), name)
    f.argtypes = argtypes
    f.restype = restype
    return f


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise SynError(rc, lib().syn_last_error().decode())


def loaded_path() -> str:
    return LIB_PATH
