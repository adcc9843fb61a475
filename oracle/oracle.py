"""ctypes bindings of the C oracle (oracle/oracle.c) and of the reference ggml build.

TEST INFRASTRUCTURE ONLY: what the HIP kernels are compared against, and the "port"
CPU baseline bench.py times.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import it.  Each function mirrors the C function of the same name minus the `or_`
prefix; the C file cites the reference function each one restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libggmlref.so")
MOE_REF_LIB = os.path.join(HERE, "_ref", "libmoeref.so")

F32, F16, Q4_0, Q8_0, Q4_K, BF16 = 0, 1, 2, 8, 12, 30
ACT_F32, ACT_Q8_0, ACT_Q8K = 0, 1, 2
BLOCK_ELEMS = {F16: 1, BF16: 1, Q8_0: 32, Q4_0: 32, Q4_K: 256}
BLOCK_BYTES = {F16: 2, BF16: 2, Q8_0: 34, Q4_0: 18, Q4_K: 144}
ACT_KIND = {F16: ACT_F32, BF16: ACT_F32, Q8_0: ACT_Q8_0, Q4_0: ACT_Q8_0, Q4_K: ACT_Q8K}

_lib = None
_ref = None
_moe_ref = None


def build() -> None:
    """Compile liboracle.so (and _ref/ where the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference/third_party/ggml"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        vp, sz, i32, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint64
        L.or_f16_bits.restype = C.c_uint16
        L.or_f16_bits.argtypes = [C.c_float]
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_round_bf16.restype = C.c_uint16
        L.or_round_bf16.argtypes = [C.c_float]
        L.or_exp.restype = C.c_float
        L.or_exp.argtypes = [C.c_float]
        L.or_silu.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_exp_worst_ulp.restype = C.c_double
        L.or_exp_worst_ulp.argtypes = [C.c_uint32]
        L.or_sum.restype = C.c_float
        L.or_sum.argtypes = [vp, sz]
        L.or_dot.restype = C.c_float
        L.or_dot.argtypes = [vp, vp, sz]
        L.or_dequantize.argtypes = [i32, vp, sz, vp]
        L.or_quantize.restype = C.c_long
        L.or_quantize.argtypes = [i32, vp, sz, vp]
        L.or_quantize_q8_0_blocks.argtypes = [vp, sz, i32, vp]
        L.or_quantize_q8_1_blocks.argtypes = [vp, sz, i32, vp]
        L.or_quantize_q8_k_blocks.argtypes = [vp, sz, vp]
        L.or_act_workspace_bytes.restype = sz
        L.or_act_workspace_bytes.argtypes = [i32, sz, sz]
        L.or_act_quantize.argtypes = [i32, vp, sz, sz, vp]
        L.or_gemv_ws.argtypes = [i32, vp, sz, sz, vp, vp, sz, sz, sz, vp]
        L.or_gemv.argtypes = [i32, vp, sz, sz, vp, sz, vp]
        L.or_gemv_threads.argtypes = [i32, vp, sz, sz, vp, sz, vp, i32]
        L.or_gemv_x86.argtypes = [i32, vp, sz, sz, vp, sz, vp, i32]
        L.or_moe_grouped_x86.argtypes = [i32, i32, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp, sz, vp, i32]
        L.or_gate_up_act.argtypes = [i32, vp, sz, sz, vp, sz, vp, i32]
        L.or_partition.argtypes = [i32, sz, sz, sz, vp, vp]
        L.or_rms_norm.argtypes = [vp, vp, sz, sz, C.c_float, vp]
        L.or_logits.argtypes = [i32, vp, sz, sz, vp, C.c_float, vp, sz, vp, i32]
        L.or_moe_workspace_bytes.restype = sz
        L.or_moe_workspace_bytes.argtypes = [sz, sz, sz, sz, sz]
        L.or_moe_pack.argtypes = [vp, sz, sz, sz, vp, vp]
        L.or_moe_grouped.argtypes = [i32, i32, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp, sz, vp, i32]
        L.or_moe_route.argtypes = [vp, vp, sz, sz, sz, sz, i32, vp, vp, vp]
        L.or_moe_combine.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        L.or_moe_combine_ranked.argtypes = [vp, vp, vp, sz, sz, sz, sz, vp]
        L.or_moe_assign.argtypes = [vp, C.c_uint32, vp, C.c_uint32, C.c_uint32, u64, C.c_uint32, vp]
        L.or_moe_assign.restype = None
        L.or_moe_doorbell.argtypes = [vp, sz, sz, C.c_uint32, vp, C.c_uint32, C.c_uint32, vp]
        L.or_moe_doorbell.restype = i32
        L.or_normal_f32.argtypes = [u64, C.c_float, vp, sz]
        L.or_fnv1a.restype = u64
        L.or_fnv1a.argtypes = [vp, sz]
        L.or_num_threads_default.restype = i32
        _lib = L
    return _lib


def moe_ref_lib():
    """The reference's split rule and doorbell headers compiled (oracle/_ref), or None."""
    global _moe_ref
    if _moe_ref is None and os.path.exists(MOE_REF_LIB):
        R = C.CDLL(MOE_REF_LIB)
        R.ref_moe_assign.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                     C.c_uint64, C.c_uint32, C.c_void_p]
        R.ref_doorbell_layout.argtypes = [C.c_void_p]
        R.ref_moe_assign_compare.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p]
        R.ref_moe_assign_compare.restype = C.c_int64
        _moe_ref = R
    return _moe_ref


def ref_lib():
    """The reference's own ggml quantizers (oracle/_ref), or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        R = C.CDLL(REF_LIB)
        R.ref_quantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        R.ref_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        R.ref_quantize_act.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        _ref = R
    return _ref


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- scalar helpers -------------------------------------------------------------------
def f16_bits(x: float) -> int:
    return lib().or_f16_bits(x)


def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def round_bf16(x: float) -> int:
    return lib().or_round_bf16(x)


def exp(x: float) -> float:
    return lib().or_exp(x)


def exp_worst_ulp(step: int) -> float:
    return lib().or_exp_worst_ulp(step)


def silu(x: float) -> float:
    return lib().or_silu(x)


def fsum(xs) -> float:
    xs = _f32(xs)
    return lib().or_sum(_p(xs), xs.size)


def fdot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    assert a.size == b.size
    return lib().or_dot(_p(a), _p(b), a.size)


# ---- quantizers -----------------------------------------------------------------------
def row_bytes(ty: int, k: int) -> int:
    return k // BLOCK_ELEMS[ty] * BLOCK_BYTES[ty]


def quantize(ty: int, x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(row_bytes(ty, x.size), dtype=np.uint8)
    n = lib().or_quantize(ty, _p(x), x.size, _p(out))
    if n < 0:
        raise ValueError("quantize refused")
    return out


def dequantize(ty: int, src) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8).ravel()
    out = np.zeros(src.size // BLOCK_BYTES[ty] * BLOCK_ELEMS[ty], dtype=np.float32)
    if lib().or_dequantize(ty, _p(src), src.size, _p(out)):
        raise ValueError("dequantize refused")
    return out


def q8_0_blocks(x, path: int) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    assert lib().or_quantize_q8_0_blocks(_p(x), x.size, path, _p(out)) == 0
    return out


def q8_1_blocks(x, path: int) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32 * 36, dtype=np.uint8)
    assert lib().or_quantize_q8_1_blocks(_p(x), x.size, path, _p(out)) == 0
    return out


def q8_k_blocks(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(x.size // 256 * 292, dtype=np.uint8)
    assert lib().or_quantize_q8_k_blocks(_p(x), x.size, _p(out)) == 0
    return out


def act_workspace_bytes(kind: int, rows: int, k: int) -> int:
    return lib().or_act_workspace_bytes(kind, rows, k)


def act_quantize(kind: int, x, rows: int, k: int):
    """Returns (d f32[blocks], sums i32[rows*k/32] or empty, codes i8[rows*k])."""
    x = _f32(x).ravel()
    nb = act_workspace_bytes(kind, rows, k)
    ws = np.zeros(max(nb, 4), dtype=np.uint8)
    assert lib().or_act_quantize(kind, _p(x), rows, k, _p(ws)) == 0
    n = rows * k
    if kind == ACT_Q8_0:
        ns, nm = n // 32, 0
    elif kind == ACT_Q8K:
        ns, nm = n // 256, n // 32
    else:
        return None
    d = ws[: 4 * ns].view(np.float32).copy()
    sums = ws[4 * ns : 4 * (ns + nm)].view(np.int32).copy()
    codes = ws[4 * (ns + nm) : 4 * (ns + nm) + n].view(np.int8).copy()
    return d, sums, codes


# ---- GEMV ----------------------------------------------------------------------------------
def gemv(ty: int, w, n_out: int, k: int, x, rows: int, threads: int = 1, level: int = 0) -> np.ndarray:
    """level 0: the portable kernels (what the GPU outputs are compared with); 1: the reference's
    x86 level (8-row groups, AVX2 block sums), the same bits, timed as the CPU baseline."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32(x).ravel()
    assert w.size == n_out * row_bytes(ty, k) and x.size >= rows * k
    y = np.full(rows * n_out, np.nan, dtype=np.float32)
    fn = lib().or_gemv_x86 if level == 1 else lib().or_gemv_threads
    if fn(ty, _p(w), n_out, k, _p(x), rows, _p(y), threads):
        raise ValueError("gemv refused")
    return y.reshape(rows, n_out)


def gate_up_act(ty: int, w, n_out: int, k: int, x, rows: int, threads: int = 1) -> np.ndarray:
    """GateUpAct{Silu}: w holds 2 n_out rows, gate then up (oracle.c or_gate_up_act)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32(x).ravel()
    assert w.size == 2 * n_out * row_bytes(ty, k) and x.size >= rows * k
    y = np.full(rows * n_out, np.nan, dtype=np.float32)
    if lib().or_gate_up_act(ty, _p(w), n_out, k, _p(x), rows, _p(y), threads):
        raise ValueError("gate_up_act refused")
    return y.reshape(rows, n_out)


def rms_norm(x, g, eps: float) -> np.ndarray:
    """RmsNorm of each row of x [rows, n] with weight g [n] (oracle.c or_rms_norm)."""
    x = _f32(x)
    rows, n = x.shape
    g = _f32(g).ravel()
    assert g.size == n
    y = np.full((rows, n), np.nan, dtype=np.float32)
    assert lib().or_rms_norm(_p(x), _p(g), rows, n, eps, _p(y)) == 0
    return y


def logits(ty: int, head, vocab: int, hidden: int, g, eps: float, x, rows: int, threads: int = 1):
    """Logits: each row of x normalised by (g, eps), then the head [vocab, hidden] as Gemv."""
    head = np.ascontiguousarray(head, dtype=np.uint8)
    x, g = _f32(x).ravel(), _f32(g).ravel()
    assert head.size == vocab * row_bytes(ty, hidden) and g.size == hidden and x.size >= rows * hidden
    y = np.full(rows * vocab, np.nan, dtype=np.float32)
    if lib().or_logits(ty, _p(head), vocab, hidden, _p(g), eps, _p(x), rows, _p(y), threads):
        raise ValueError("logits refused")
    return y.reshape(rows, vocab)


def partition(ty: int, n_out: int, k: int, parts: int):
    s = np.zeros(max(parts, 1), dtype=np.uint64)
    e = np.zeros(max(parts, 1), dtype=np.uint64)
    lib().or_partition(ty, n_out, k, parts, _p(s), _p(e))
    return list(zip(s.tolist(), e.tolist()))


# ---- MoE -------------------------------------------------------------------------------
def moe_pack(ids, n_experts: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows, top_k = ids.shape
    offsets = np.zeros(n_experts + 1, dtype=np.uint32)
    slots = np.zeros(rows * top_k, dtype=np.uint32)
    if lib().or_moe_pack(_p(ids), rows, top_k, n_experts, _p(offsets), _p(slots)):
        raise ValueError("expert id out of range")
    return offsets, slots


def moe_grouped(gate_ty, down_ty, n_experts, top_k, hidden, inter, gate, up, down, x, ids,
                site=None, threads: int = 1, out=None, level: int = 0) -> np.ndarray:
    x = _f32(x)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows = ids.shape[0]
    if out is None:
        out = np.full(rows * top_k * hidden, np.nan, dtype=np.float32)
    gate, up, down = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    s = None if site is None else np.ascontiguousarray(site, dtype=np.int32)
    fn = lib().or_moe_grouped_x86 if level == 1 else lib().or_moe_grouped
    rc = fn(gate_ty, down_ty, n_experts, top_k, hidden, inter, _p(gate), _p(up), _p(down), _p(x), _p(ids), _p(s),
            rows, _p(out), threads)
    if rc:
        raise ValueError(f"moe_grouped refused ({rc})")
    return out.reshape(rows, top_k, hidden)


def moe_route(router, x, n_experts: int, top_k: int, renormalize: bool = True):
    router, x = _f32(router), _f32(x)
    rows, hidden = x.shape
    ids = np.zeros((rows, top_k), dtype=np.int32)
    w = np.zeros((rows, top_k), dtype=np.float32)
    probs = np.zeros((rows, n_experts), dtype=np.float32)
    if lib().or_moe_route(_p(router), _p(x), rows, hidden, n_experts, top_k, int(renormalize),
                          _p(ids), _p(w), _p(probs)):
        raise ValueError("moe_route refused")
    return ids, w, probs


def moe_combine(out, ids, w) -> np.ndarray:
    out, w = _f32(out), _f32(w)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows, top_k, hidden = out.shape
    y = np.zeros((rows, hidden), dtype=np.float32)
    assert lib().or_moe_combine(_p(out), _p(ids), _p(w), rows, top_k, hidden, _p(y)) == 0
    return y


def moe_combine_ranked(out, w, shared=()) -> np.ndarray:
    """MoeCombine as the IR binds it: slots in rank order, then each shared output [rows, hidden]."""
    out, w = _f32(out), _f32(w)
    rows, top_k, hidden = out.shape
    sh = np.ascontiguousarray(np.stack([_f32(a).reshape(rows, hidden) for a in shared])) if len(shared) \
        else np.zeros((0, rows, hidden), np.float32)
    y = np.zeros((rows, hidden), dtype=np.float32)
    assert lib().or_moe_combine_ranked(_p(out), _p(w), _p(sh) if len(shared) else None, len(shared), rows,
                                       top_k, hidden, _p(y)) == 0
    return y


# ---- the residency split ------------------------------------------------------------------
# syn_route_slot of moe_doorbell.h
ROUTE_SLOT = np.dtype([("expert", "<u2"), ("tokens", "<u2"), ("cache_slot", "<u4")])
MOE_MISS, MOE_HIT, MOE_CPU = 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFE
DOORBELL_HEADER = 8


def route_slots(entries) -> np.ndarray:
    """[(expert, tokens, cache_slot), ...] as syn_route_slot records."""
    return np.array([tuple(e) for e in entries], dtype=ROUTE_SLOT)


def moe_assign(route, eligible, n_experts: int, b_copy: int, expert_bytes: int,
               copy_slots: int) -> np.ndarray:
    """The split rule: one u32 code per route entry (MOE_HIT, MOE_CPU or a copy-slot index)."""
    route = np.ascontiguousarray(route, dtype=ROUTE_SLOT)
    words = np.ascontiguousarray(eligible if eligible is not None else [], dtype=np.uint32)
    out = np.zeros(len(route), np.uint32)
    lib().or_moe_assign(_p(route), len(route), _p(words) if words.size else None, n_experts,
                        b_copy, expert_bytes, copy_slots, _p(out))
    return out


def moe_doorbell(ids, n_experts: int, max_union: int, slot_of=None, seq: int = 0):
    """The doorbell layer's header and route part (bytes), or None when refused."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows, top_k = ids.shape
    layer = np.zeros(DOORBELL_HEADER + 8 * max_union, np.uint8)
    so = None if slot_of is None else np.ascontiguousarray(slot_of, dtype=np.uint32)
    rc = lib().or_moe_doorbell(_p(ids), rows, top_k, n_experts, _p(so) if so is not None else None,
                               seq, max_union, _p(layer))
    return None if rc else layer


# ---- data ------------------------------------------------------------------------------
def normal(seed: int, sigma: float, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().or_normal_f32(seed, sigma, _p(out), n)
    return out


def fnv1a(b) -> int:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    return lib().or_fnv1a(_p(b), b.size)


def num_threads_default() -> int:
    return lib().or_num_threads_default()
