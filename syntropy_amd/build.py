"""Builds libsyntropy_hip.so and libsyntropy_provider.so for gfx950 in-tree with hipcc.

    python -m syntropy_amd.build          # compile every source, link the library

Two libraries, both C-ABI only and linking nothing of PyTorch: libsyntropy_hip.so (the
kernels' entry points, include/syntropy_hip.h) and libsyntropy_provider.so (the same kernels
behind the provider-library boundary, include/syntropy_provider.h).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsyntropy_hip.so")
# The provider library: the same kernels behind the one symbol syntropy_provider_entry_v1
# (include/syntropy_provider.h), everything else local, linked -Bsymbolic.
PROVIDER_LIB = os.path.join(HERE, "libsyntropy_provider.so")
PROVIDER_MAP = os.path.join(HERE, "provider.map")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Numerics: one IEEE operation per source operation (no contraction), correctly rounded F32
# division and square root, F32 denormals kept.  Packed-F32 instructions are disabled.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


# Per-source additions.  gemv_split.hip: the matrix products' results go straight to VGPRs (no
# accumulation-register reads in the F32 epilogue that follows every product).
FILE_FLAGS = {"gemv_split.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def _link(out: str, objs, extra=()) -> None:
    tmp = out + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *extra],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {out} failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


# Host code under AddressSanitizer and UndefinedBehaviorSanitizer (each flag for the host pass
# only: the kernels' device code is built as always).  The libraries this gives resolve the
# sanitizer runtime from the program that loads them (tests/sanitize/host_paths.cpp).
SANITIZE_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
                 "-Xarch_host", "-g"]


def build_host_sanitized(out_dir: str, jobs: int = 8) -> tuple:
    """Both libraries with sanitized host code, into out_dir; returns their paths."""
    obj_dir = os.path.join(out_dir, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()

    def one(src):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        lang = ["-x", "hip"] if src.endswith(".cpp") else FILE_FLAGS.get(os.path.basename(src), [])
        r = subprocess.run([HIPCC, *FLAGS, *SANITIZE_HOST, *lang, "-c", src, "-o", obj], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(one, srcs))
    provider = [o for o in objs if os.path.basename(o).startswith("provider.")]
    kernels = [o for o in objs if o not in provider]
    lib = os.path.join(out_dir, os.path.basename(LIB))
    plib = os.path.join(out_dir, os.path.basename(PROVIDER_LIB))
    _link(lib, kernels)
    _link(plib, objs, [f"-Wl,--version-script={PROVIDER_MAP}", "-Wl,-Bsymbolic"])
    return lib, plib


def build(jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    provider = [o for o in objs if os.path.basename(o).startswith("provider.")]
    kernels = [o for o in objs if o not in provider]
    _link(LIB, kernels)
    _link(PROVIDER_LIB, objs, [f"-Wl,--version-script={PROVIDER_MAP}", "-Wl,-Bsymbolic"])
    shutil.rmtree(OBJ, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build())
