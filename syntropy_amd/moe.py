"""The MoE layer on the MI355X, mirroring the reference CPU provider's `moe` module
(crates/kernels-cpu/src/moe.rs) and the MoeRoute / MoeCombine ops (crates/kernels/src/op/kind.rs,
crates/graph/src/blocks/ffn.rs:127-200): route -> pack -> grouped expert FFN -> combine, every
step a HIP kernel behind the C ABI.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import call
from .gemv import GemvError, WeightType, _stream


@dataclass(frozen=True)
class MoeShape:
    """The layer's MoE shape: MoeGrouped's dims [n_experts, top_k, hidden, inter]
    (crates/kernels-cpu/src/moe.rs:89-101)."""

    n_experts: int
    top_k: int
    hidden: int
    inter: int


class MoeError(ValueError):
    """Why a MoE call refused its inputs (moe.rs:148-166).  A refused call writes nothing."""


LAYOUT_SOURCE, LAYOUT_TILE64 = 0, 3


@dataclass
class Experts:
    """One layer's experts stacked by expert (ffn_gate_exps, ffn_up_exps, ffn_down_exps):
    gate/up [n_experts][inter, hidden], down [n_experts][hidden, inter], uint8 device tensors of
    one weight type, in GGUF block layout (`layout` 0) or, for Q4_K, TILE64 (3: each run of 64
    rows stored super-block-major; `tile64` makes it)."""

    ty: WeightType
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    layout: int = LAYOUT_SOURCE

    def check(self, s: MoeShape):
        ty = WeightType(self.ty)
        if ty not in (WeightType.Q4K, WeightType.Q8_0):
            raise MoeError("MoeGrouped takes Q4_K or Q8_0 experts (crates/kernels-cpu/src/moe/entry.rs:50-55)")
        if self.layout not in (LAYOUT_SOURCE, LAYOUT_TILE64) or (self.layout == LAYOUT_TILE64 and ty != WeightType.Q4K):
            raise MoeError(f"experts of {ty.name} in layout {self.layout} (0, or 3 for Q4_K)")
        need = s.n_experts * s.inter * (s.hidden // ty.block_elems()) * ty.block_bytes()
        for name, t in (("gate", self.gate), ("up", self.up), ("down", self.down)):
            if t.dtype != torch.uint8 or t.numel() != need:
                raise MoeError(f"`{name}` holds {t.numel()} bytes, the experts need {need}")


def tile64_repack(w: torch.Tensor, k: int, inverse: bool = False, stream=None) -> torch.Tensor:
    """Q4_K rows of k values, whole runs of 64 rows, GGUF order -> TILE64 (or back)."""
    if w.dtype != torch.uint8 or not w.is_contiguous():
        raise MoeError("the rows must be contiguous uint8")
    out = torch.empty_like(w)
    call("syn_q4k_tile64_repack", w.data_ptr(), out.data_ptr(), w.numel(), k, 1 if inverse else 0, _stream(stream))
    return out


def tile64(experts: Experts, s: MoeShape, stream=None) -> Experts:
    """The experts repacked to TILE64 (new tensors; the GGUF ones are left as they are)."""
    experts.check(s)
    if experts.layout == LAYOUT_TILE64:
        return experts
    return Experts(experts.ty, tile64_repack(experts.gate, s.hidden, stream=stream),
                   tile64_repack(experts.up, s.hidden, stream=stream),
                   tile64_repack(experts.down, s.inter, stream=stream), LAYOUT_TILE64)


def route(router: torch.Tensor, x: torch.Tensor, top_k: int, renormalize: bool = True,
          probs: bool = False, stream=None):
    """MoeRoute{Softmax}: (ids I32 [rows, k], weights F32 [rows, k][, probs])."""
    n_experts, hidden = router.shape
    rows = x.shape[0]
    ids = torch.empty(rows, top_k, dtype=torch.int32, device=x.device)
    w = torch.empty(rows, top_k, dtype=torch.float32, device=x.device)
    p = torch.empty(rows, n_experts, dtype=torch.float32, device=x.device)
    call("syn_moe_route", router.data_ptr(), x.data_ptr(), rows, hidden, n_experts, top_k,
         int(renormalize), ids.data_ptr(), w.data_ptr(), p.data_ptr(), _stream(stream))
    return (ids, w, p) if probs else (ids, w)


def pack(ids: torch.Tensor, n_experts: int, stream=None):
    """(offsets u32 [E+1], slots u32 [rows*k], err u32 [2]) as int32 tensors: err[0] = bad id,
    err[1] = the largest expert's slot count."""
    rows, top_k = ids.shape
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=ids.device)
    slots = torch.empty(rows * top_k, dtype=torch.int32, device=ids.device)
    err = torch.empty(2, dtype=torch.int32, device=ids.device)
    call("syn_moe_pack", ids.data_ptr(), rows, top_k, n_experts, offsets.data_ptr(),
         slots.data_ptr(), err.data_ptr(), _stream(stream))
    return offsets, slots, err


def workspace_bytes(s: MoeShape, rows: int, ty: WeightType = WeightType.Q4K) -> int:
    out = C.c_uint64()
    call("syn_moe_grouped_workspace_bytes", int(ty), s.n_experts, s.top_k, s.hidden, s.inter, rows,
         C.byref(out))
    return out.value


def moe_grouped(s: MoeShape, experts: Experts, x: torch.Tensor, ids: torch.Tensor,
                out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                status: torch.Tensor | None = None, stream=None,
                site: torch.Tensor | None = None) -> torch.Tensor:
    """MoeGrouped (moe.rs:402-518): out F32 [rows, top_k, hidden], the same bits in either expert
    layout.  site (I32 [n_experts],
    optional): experts marked zero are not computed and their slots of out keep their values
    (moe/entry.rs:13-16, 297-300)."""
    experts.check(s)
    rows = ids.shape[0]
    if ids.shape != (rows, s.top_k) or ids.dtype != torch.int32:
        raise MoeError("ids must be I32 [rows, top_k]")
    if x.dtype != torch.float32 or x.numel() < rows * s.hidden or not x.is_contiguous():
        raise MoeError("x must be contiguous F32 [rows, hidden]")
    if site is not None and (site.dtype != torch.int32 or site.numel() != s.n_experts
                             or not site.is_contiguous() or site.device != x.device):
        raise MoeError("site must be contiguous I32 [n_experts] on x's device")
    if out is None:
        out = torch.empty(rows, s.top_k, s.hidden, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = torch.empty(max(workspace_bytes(s, rows, WeightType(experts.ty)), 256), dtype=torch.uint8,
                         device=x.device)
    call("syn_moe_grouped_layout", experts.layout, int(experts.ty), experts.gate.data_ptr(), experts.up.data_ptr(),
         experts.down.data_ptr(), experts.gate.numel(), s.n_experts, s.top_k, s.hidden, s.inter,
         x.data_ptr(), ids.data_ptr(), site.data_ptr() if site is not None else None, rows,
         out.data_ptr(), ws.data_ptr(), ws.numel(),
         status.data_ptr() if status is not None else None, _stream(stream))
    return out


def combine(out: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, y: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """MoeCombine: y F32 [rows, hidden] (moe/tests.rs:541-556)."""
    rows, top_k, hidden = out.shape
    if y is None:
        y = torch.empty(rows, hidden, dtype=torch.float32, device=out.device)
    call("syn_moe_combine", out.data_ptr(), ids.data_ptr(), w.data_ptr(), rows, top_k, hidden,
         y.data_ptr(), _stream(stream))
    return y


def combine_ranked(out: torch.Tensor, w: torch.Tensor, shared=(), y: torch.Tensor | None = None,
                   stream=None) -> torch.Tensor:
    """MoeCombine as the graph binds it (crates/graph/src/blocks/ffn.rs:189-200): the slots of out
    F32 [rows, top_k, hidden] in rank order, then each shared output F32 [rows, hidden]."""
    rows, top_k, hidden = out.shape
    if len(shared) > 8:
        raise MoeError("at most 8 shared outputs")
    for t in shared:
        if t.shape != (rows, hidden) or t.dtype != torch.float32 or not t.is_contiguous():
            raise MoeError("each shared output is contiguous F32 [rows, hidden]")
    if y is None:
        y = torch.empty(rows, hidden, dtype=torch.float32, device=out.device)
    ptrs = (C.c_void_p * max(1, len(shared)))(*[t.data_ptr() for t in shared])
    call("syn_moe_combine_ranked", out.data_ptr(), w.data_ptr(), len(shared), ptrs if shared else None, rows,
         top_k, hidden, y.data_ptr(), _stream(stream))
    return y


class MoeLayer:
    """route -> MoeGrouped -> MoeCombine for one layer, as the graph binds them (the combine in
    rank order), with its workspace held."""

    def __init__(self, s: MoeShape, router: torch.Tensor, experts: Experts, max_rows: int):
        self.s, self.router, self.experts = s, router, experts
        self.ws = torch.empty(max(workspace_bytes(s, max_rows, WeightType(experts.ty)), 256), dtype=torch.uint8,
                              device=router.device)
        self.max_rows = max_rows

    def __call__(self, x: torch.Tensor, stream=None):
        rows = x.shape[0]
        if rows > self.max_rows:
            raise MoeError(f"{rows} rows above the layer's {self.max_rows}")
        ids, w = route(self.router, x, self.s.top_k, True, stream=stream)
        out = moe_grouped(self.s, self.experts, x, ids, ws=self.ws, stream=stream)
        return combine_ranked(out, w, stream=stream), ids, w, out


# ---- the residency split (doorbell layer, split rule, site masks) ------------------------------
HIT, COPY, CPU = 0, 1, 2  # site-mask classes


def doorbell_bytes(max_union: int) -> int:
    """Header and route part of a doorbell layer (moe_doorbell.h: 8 + 8 * MAX_UNION)."""
    return 8 + 8 * max_union


def doorbell(ids: torch.Tensor, n_experts: int, max_union: int, slot_of: torch.Tensor | None = None,
             seq: int = 0, step_desc: torch.Tensor | None = None, layer: torch.Tensor | None = None,
             status: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """The pass's doorbell layer (RFC-0040 3.4): seq, then one route entry per distinct expert of
    ids, ascending.  Returns the layer as uint8 [8 + 8 * max_union]."""
    rows, top_k = ids.shape
    if layer is None:
        layer = torch.zeros(doorbell_bytes(max_union), dtype=torch.uint8, device=ids.device)
    if layer.numel() < doorbell_bytes(max_union):
        raise MoeError("the layer is shorter than its route part")
    call("syn_moe_doorbell", ids.data_ptr(), rows, top_k, n_experts,
         slot_of.data_ptr() if slot_of is not None else None,
         step_desc.data_ptr() if step_desc is not None else None, seq, layer.data_ptr(), max_union,
         status.data_ptr() if status is not None else None, _stream(stream))
    return layer


def assign(route: torch.Tensor, n_route: int, eligible: torch.Tensor | None, n_experts: int, b_copy: int,
           expert_bytes: int, copy_slots: int, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """The split rule (moe_assign.h): one code per route entry, as int32 (HIT = -1, CPU = -2)."""
    if out is None:
        out = torch.empty(max(n_route, 1), dtype=torch.int32, device=route.device)
    call("syn_moe_assign", route.data_ptr(), n_route, eligible.data_ptr() if eligible is not None else None,
         n_experts, b_copy, expert_bytes, copy_slots, out.data_ptr(), _stream(stream))
    return out


def assign_layer(layer: torch.Tensor, max_union: int, eligible: torch.Tensor | None, n_experts: int,
                 b_copy: torch.Tensor, expert_bytes: int, copy_slots: int, out: torch.Tensor | None = None,
                 stream=None) -> torch.Tensor:
    """The split rule over a doorbell layer, n_route and b_copy read on the device."""
    if out is None:
        out = torch.empty(max(max_union, 1), dtype=torch.int32, device=layer.device)
    call("syn_moe_assign_layer", layer.data_ptr(), max_union,
         eligible.data_ptr() if eligible is not None else None, n_experts, b_copy.data_ptr(), expert_bytes,
         copy_slots, out.data_ptr(), _stream(stream))
    return out


def site_mask(layer: torch.Tensor, max_union: int, codes: torch.Tensor, n_experts: int, which: int,
              site: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """I32 [n_experts]: 1 for the route's experts whose code is of class `which` (HIT, COPY, CPU)."""
    if site is None:
        site = torch.empty(n_experts, dtype=torch.int32, device=layer.device)
    call("syn_moe_site_mask", layer.data_ptr(), max_union, codes.data_ptr(), n_experts, which, site.data_ptr(),
         _stream(stream))
    return site


__all__ = ["MoeShape", "MoeError", "Experts", "LAYOUT_SOURCE", "LAYOUT_TILE64", "tile64", "tile64_repack", "route", "pack", "workspace_bytes", "moe_grouped",
           "combine", "combine_ranked", "MoeLayer", "GemvError", "doorbell", "doorbell_bytes", "assign", "assign_layer",
           "site_mask", "HIT", "COPY", "CPU"]
