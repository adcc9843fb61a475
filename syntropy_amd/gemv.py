"""Decode GEMV on the MI355X, mirroring the reference CPU provider's `gemv` module
(crates/kernels-cpu/src/gemv.rs, gemv/act.rs, gemv/entry.rs): the same names, argument
meaning and refusals, over device tensors.  Every call runs the HIP kernels through the C ABI;
there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

import torch

from ._lib import SynError, call, lib


class WeightType(IntEnum):
    """A weight type this module computes (gemv.rs:87-151), by ggml type id."""

    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4K = 12
    BF16 = 30

    def block_elems(self) -> int:
        return {WeightType.F16: 1, WeightType.BF16: 1, WeightType.Q4K: 256}.get(self, 32)

    def block_bytes(self) -> int:
        return {WeightType.F16: 2, WeightType.BF16: 2, WeightType.Q4_0: 18, WeightType.Q8_0: 34,
                WeightType.Q4K: 144}[self]

    def act(self) -> str:
        """The activation block a product over this type quantizes to (gemv.rs:145-151); F16 and
        BF16 products take the F32 activations as they are."""
        if self in (WeightType.F16, WeightType.BF16):
            return "F32"
        return "Q8K" if self is WeightType.Q4K else "Q8_0"


class GemvError(ValueError):
    """Why a GEMV call refused its inputs (gemv.rs:226-279).  A refused call writes nothing."""

    def __init__(self, kind: str, msg: str):
        super().__init__(f"Gemv: {msg}")
        self.kind = kind


LAYOUT_SOURCE, LAYOUT_X8, LAYOUT_SPLIT = 0, 1, 2


@dataclass
class Weights:
    """`n_out` rows of `k_in` weights of type `ty` in GGUF block layout, in device memory
    (gemv.rs:157-224).  `bytes` is a uint8 device tensor holding exactly the matrix; `layout` is
    LAYOUT_SOURCE (the GGUF order), for Q4_K LAYOUT_X8, for Q8_0 and Q4_0 LAYOUT_SPLIT (see
    repack)."""

    ty: WeightType
    bytes: torch.Tensor
    n_out: int
    k_in: int
    layout: int = LAYOUT_SOURCE

    def __post_init__(self):
        self.ty = WeightType(self.ty)
        if self.k_in % self.ty.block_elems():
            raise GemvError("RowLength", f"a row of {self.k_in} weights is not whole "
                            f"{self.ty.block_elems()}-weight {self.ty.name} blocks")
        need = self.row_bytes() * self.n_out
        if self.bytes.dtype != torch.uint8 or self.bytes.numel() != need:
            raise GemvError("Len", f"`weights` holds {self.bytes.numel()} values, the op needs {need}")

    def row_bytes(self) -> int:
        return self.k_in // self.ty.block_elems() * self.ty.block_bytes()


def workspace_bytes(ty: WeightType, rows: int, k: int) -> int:
    """Scratch bytes of one call's quantized activations (act.rs:108-111; the provider's own
    layout: codes, scales, 32-value sums)."""
    out = C.c_uint64()
    call("syn_gemv_workspace_bytes", int(ty), rows, k, C.byref(out))
    return out.value


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


def _check_x(x: torch.Tensor, rows: int, k: int):
    if not (x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()):
        raise GemvError("Len", "x must be a contiguous F32 device tensor")
    if x.numel() < rows * k:
        raise GemvError("Len", f"`x` holds {x.numel()} values, the op needs {rows * k}")


def new_workspace(ty: WeightType, rows: int, k: int, device="cuda") -> torch.Tensor:
    return torch.empty(max(workspace_bytes(ty, rows, k), 256), dtype=torch.uint8, device=device)


def quantize_into(ty: WeightType, x: torch.Tensor, rows: int, k: int, ws: torch.Tensor,
                  stream=None) -> None:
    """Quantizes the first `rows` rows of x (k values each) into `ws` (act.rs:122-167)."""
    ty = WeightType(ty)
    if k % ty.block_elems():
        raise GemvError("Activations", "k is not whole activation blocks")
    _check_x(x, rows, k)
    call("syn_act_quantize", int(ty), x.data_ptr(), rows, k, ws.data_ptr(), ws.numel(), _stream(stream))


def gemv_quantized(w: Weights, ws: torch.Tensor, rows: int, y: torch.Tensor, stream=None) -> None:
    """y[r][o] for every row r < rows and every output o (gemv.rs:435-492)."""
    need = rows * w.n_out
    if y.numel() < need:
        raise GemvError("Len", f"`y` holds {y.numel()} values, the op needs {need}")
    call("syn_gemv_quantized_layout", w.layout, int(w.ty), w.bytes.data_ptr(), w.bytes.numel(), w.n_out,
         w.k_in, ws.data_ptr(), ws.numel(), rows, y.data_ptr(), _stream(stream))


def repack(w: Weights, layout: int | None = None, stream=None) -> Weights:
    """The matrix in another layout (a permutation of its bytes, crates/kernels/src/provider.rs:
    326-336 repack): LAYOUT_X8 stores each run of eight Q4_K super-blocks chunk-major, so the
    decode kernel reads whole 128-byte lines; LAYOUT_SPLIT stores every Q8_0 / Q4_0 block's codes
    first and every block's F16 scale after them, so the codes stream in 16-byte loads."""
    if layout is None:
        layout = LAYOUT_X8 if w.ty is WeightType.Q4K else LAYOUT_SPLIT
    if w.layout != LAYOUT_SOURCE:
        raise GemvError("Activations", "repack takes weights in the source layout")
    out = torch.empty_like(w.bytes)
    if w.ty is WeightType.Q4K and layout == LAYOUT_X8:
        call("syn_q4k_repack", layout, w.bytes.data_ptr(), out.data_ptr(), w.bytes.numel(), 0, _stream(stream))
    elif w.ty in (WeightType.Q8_0, WeightType.Q4_0) and layout == LAYOUT_SPLIT:
        call("syn_split_repack", layout, int(w.ty), w.bytes.data_ptr(), out.data_ptr(), w.bytes.numel(), 0,
             _stream(stream))
    else:
        raise GemvError("Activations", "repack takes Q4_K to LAYOUT_X8 and Q8_0 / Q4_0 to LAYOUT_SPLIT")
    return Weights(w.ty, out, w.n_out, w.k_in, layout)


def gemv(w: Weights, x: torch.Tensor, rows: int, y: torch.Tensor | None = None,
         ws: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """The Gemv op (gemv/entry.rs:167-247): quantize x F32 [rows, k_in], then
    y F32 [rows, n_out] = W x, bit-identical to the reference CPU provider."""
    _check_x(x, rows, w.k_in)
    if y is None:
        y = torch.empty(rows, w.n_out, dtype=torch.float32, device=x.device)
    elif y.numel() < rows * w.n_out:
        raise GemvError("Len", f"`y` holds {y.numel()} values, the op needs {rows * w.n_out}")
    if w.layout != LAYOUT_SOURCE:
        if ws is None:
            need = C.c_uint64()
            call("syn_gemv_layout_workspace_bytes", w.layout, int(w.ty), rows, w.k_in, C.byref(need))
            ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=x.device)
        call("syn_gemv_layout", w.layout, int(w.ty), w.bytes.data_ptr(), w.bytes.numel(), w.n_out, w.k_in,
             x.data_ptr(), rows, y.data_ptr(), ws.data_ptr(), ws.numel(), _stream(stream))
        return y
    if ws is None:
        ws = new_workspace(w.ty, rows, w.k_in, x.device)
    call("syn_gemv", int(w.ty), w.bytes.data_ptr(), w.bytes.numel(), w.n_out, w.k_in,
         x.data_ptr(), rows, y.data_ptr(), ws.data_ptr(), ws.numel(), _stream(stream))
    return y


def gate_up_act(w: Weights, x: torch.Tensor, rows: int, y: torch.Tensor | None = None,
                stream=None) -> torch.Tensor:
    """GateUpAct{Silu} (crates/kernels/src/reference/linear.rs:75-112): `w` stacks the gate rows
    then the up rows (w.n_out = 2 n), y F32 [rows, n] = silu(gate x) * (up x), each dot the
    Gemv value, silu with the reference's software exp, the product rounded once."""
    if w.n_out % 2:
        raise GemvError("Len", f"a stacked gate/up matrix has an even row count, not {w.n_out}")
    n = w.n_out // 2
    _check_x(x, rows, w.k_in)
    if y is None:
        y = torch.empty(rows, n, dtype=torch.float32, device=x.device)
    elif y.numel() < rows * n:
        raise GemvError("Len", f"`y` holds {y.numel()} values, the op needs {rows * n}")
    need = C.c_uint64()
    call("syn_gate_up_act_workspace_bytes", w.layout, int(w.ty), rows, n, w.k_in, C.byref(need))
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=x.device)
    call("syn_gate_up_act", w.layout, int(w.ty), w.bytes.data_ptr(), w.bytes.numel(), n, w.k_in,
         x.data_ptr(), rows, y.data_ptr(), ws.data_ptr(), ws.numel(), _stream(stream))
    return y


def rms_norm(x: torch.Tensor, g: torch.Tensor, eps: float, rows: int, y: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """RmsNorm of each row of x F32 [rows, n] (crates/kernels/src/reference/norm.rs:39-47)."""
    n = g.numel()
    _check_x(x, rows, n)
    if y is None:
        y = torch.empty(rows, n, dtype=torch.float32, device=x.device)
    call("syn_rms_norm", x.data_ptr(), g.data_ptr(), rows, n, C.c_float(eps), y.data_ptr(), _stream(stream))
    return y


def logits(head: Weights, g: torch.Tensor, eps: float, x: torch.Tensor, rows: int,
           y: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Logits (crates/kernels/src/reference/linear.rs:118-161): each row of x [rows, hidden]
    normalised by (g, eps), then y F32 [rows, vocab] = head x as the Gemv op computes it."""
    _check_x(x, rows, head.k_in)
    if y is None:
        y = torch.empty(rows, head.n_out, dtype=torch.float32, device=x.device)
    need = C.c_uint64()
    call("syn_logits_workspace_bytes", head.layout, int(head.ty), rows, head.n_out, head.k_in, C.byref(need))
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=x.device)
    call("syn_logits", head.layout, int(head.ty), head.bytes.data_ptr(), head.bytes.numel(), head.n_out,
         head.k_in, g.data_ptr(), C.c_float(eps), x.data_ptr(), rows, y.data_ptr(), ws.data_ptr(), ws.numel(),
         _stream(stream))
    return y


class GemvBatch:
    """Up to 8 independent single-row Q4_K Gemv ops launched together (one batched Q8_K
    quantization, one grouped GEMV): each y[i] equals gemv(ws[i], x[i], 1) bit for bit.  The
    argument arrays are built once; `__call__` launches."""

    def __init__(self, weights: list[Weights], xs: list[torch.Tensor], ys: list[torch.Tensor],
                 ws: torch.Tensor | None = None):
        n = len(weights)
        if not (n == len(xs) == len(ys)) or n > 8:
            raise GemvError("Len", "GemvBatch takes up to 8 (weights, x, y) triples")
        for w, x, y in zip(weights, xs, ys):
            if w.ty is not WeightType.Q4K:
                raise GemvError("Activations", "GemvBatch takes Q4_K weights")
            _check_x(x, 1, w.k_in)
            if y.numel() < w.n_out:
                raise GemvError("Len", f"`y` holds {y.numel()} values, the op needs {w.n_out}")
        layouts = {w.layout for w in weights}
        if len(layouts) > 1:
            raise GemvError("Activations", "GemvBatch takes weights of one layout")
        self.layout = layouts.pop() if layouts else LAYOUT_SOURCE
        self.n = n
        u32 = C.c_uint32 * n
        self.k = u32(*[w.k_in for w in weights])
        self.n_out = u32(*[w.n_out for w in weights])
        self.ty = (C.c_int32 * n)(*[int(w.ty) for w in weights])
        self.w = (C.c_void_p * n)(*[w.bytes.data_ptr() for w in weights])
        self.wb = (C.c_uint64 * n)(*[w.bytes.numel() for w in weights])
        self.x = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
        self.y = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        need = C.c_uint64()
        call("syn_gemv_batch_workspace_bytes", n, self.k, C.byref(need))
        self.ws = ws if ws is not None else torch.empty(max(need.value, 256), dtype=torch.uint8,
                                                        device=xs[0].device)
        self._keep = (weights, xs, ys)

    def __call__(self, stream=None) -> None:
        call("syn_gemv_batch_layout", self.layout, self.n, self.ty, self.w, self.wb, self.n_out, self.k,
             self.x, self.y, self.ws.data_ptr(), self.ws.numel(), _stream(stream))

    def quantize(self, stream=None) -> None:
        """The first half of __call__: every x[i] to Q8_K in the held workspace."""
        call("syn_act_quantize_batch", self.n, self.k, self.x, self.ws.data_ptr(), self.ws.numel(),
             _stream(stream))

    def gemv_quantized(self, stream=None) -> None:
        """The second half: every y[i] from the workspace quantize() filled."""
        call("syn_gemv_batch_quantized_layout", self.layout, self.n, self.ty, self.w, self.wb, self.n_out,
             self.k, self.ws.data_ptr(), self.ws.numel(), self.y, _stream(stream))


def gemm_workspace(rows: int, k: int, device="cuda") -> torch.Tensor:
    """Workspace of the prefill GEMM's activations (rows x k, Q8_K in the GEMM layout)."""
    out = C.c_uint64()
    call("syn_gemm_workspace_bytes", rows, k, C.byref(out))
    return torch.empty(max(out.value, 256), dtype=torch.uint8, device=device)


def gemm_quantize_into(x: torch.Tensor, rows: int, k: int, ws: torch.Tensor, stream=None) -> None:
    """The first `rows` rows of x to Q8_K in the prefill GEMM's layout (act.rs:351-373 values)."""
    _check_x(x, rows, k)
    call("syn_gemm_act_quantize", x.data_ptr(), rows, k, ws.data_ptr(), ws.numel(), _stream(stream))


def gemm_quantized(w: Weights, ws: torch.Tensor, rows: int, y: torch.Tensor, stream=None) -> None:
    """y[r][o] for every row r < rows from a workspace gemm_quantize_into filled: the Q4_K
    matrix-core GEMM, every output the Gemv value (gemv.rs:435-547)."""
    if w.ty is not WeightType.Q4K:
        raise GemvError("Activations", "the prefill GEMM takes Q4_K weights")
    if y.numel() < rows * w.n_out:
        raise GemvError("Len", f"`y` holds {y.numel()} values, the op needs {rows * w.n_out}")
    call("syn_gemm_q4k_quantized", w.bytes.data_ptr(), w.bytes.numel(), w.n_out, w.k_in, ws.data_ptr(),
         ws.numel(), rows, y.data_ptr(), _stream(stream))


def quantize(ty: WeightType, x: torch.Tensor, stream=None) -> torch.Tensor:
    """F32 values -> GGUF blocks, byte-identical to ggml's reference quantizers
    (crates/kernels-ggml/src/lib.rs:268 quantize).  Like that wrapper, refuses non-finite
    values and magnitudes above 65504 (checked on the device, one reduction)."""
    ty = WeightType(ty)
    x = x.contiguous()
    if x.numel() % ty.block_elems():
        raise GemvError("RowLength", f"{x.numel()} values are not whole {ty.block_elems()}-value blocks")
    if x.numel() and not bool(torch.isfinite(x).all() and x.abs().max() <= 65504.0):
        raise GemvError("OutOfRange", "a value is not finite or is out of the type's range")
    out = torch.empty(x.numel() // ty.block_elems() * ty.block_bytes(), dtype=torch.uint8, device=x.device)
    call("syn_quantize", int(ty), x.data_ptr(), x.numel(), out.data_ptr(), out.numel(), _stream(stream))
    return out


def dequantize(ty: WeightType, src: torch.Tensor, stream=None) -> torch.Tensor:
    """GGUF blocks -> F32, exact (dequant.rs:195-229)."""
    ty = WeightType(ty)
    out = torch.empty(src.numel() // ty.block_bytes() * ty.block_elems(), dtype=torch.float32,
                      device=src.device)
    call("syn_dequantize", int(ty), src.data_ptr(), src.numel(), out.data_ptr(), _stream(stream))
    return out


__all__ = ["WeightType", "Weights", "GemvError", "SynError", "GemvBatch", "workspace_bytes", "quantize_into",
           "repack", "LAYOUT_SOURCE", "LAYOUT_X8", "LAYOUT_SPLIT",
           "gemv_quantized", "gemv", "quantize", "dequantize", "new_workspace", "gemm_workspace",
           "gemm_quantize_into", "gemm_quantized", "gate_up_act", "lib"]
