#!/usr/bin/env python3
"""Benchmark of the quantized-matmul path on one MI355X.

Headline workload: one Q4_K decode layer's matmuls at Llama-3-8B shapes, batch 1 (QKV
6144x4096, O 4096x4096, gate and up 14336x4096, down 4096x14336).  One step quantizes each
GEMV's F32 activation row to Q8_K and runs the five GEMVs.  Weights are N(0, 0.02) quantized by
the GPU Q4_K packer (byte-identical to ggml's), then repacked once to the X8 layout (the
provider's repack: a permutation of the bytes), in COPIES distinct copies that the steps rotate
through, so the weights come from HBM and not from the 256 MB Infinity Cache.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only PART] [--no-cpu]

Prints one JSON line: whole-step weight GB/s (value), the roofline of the GEMV kernel from HIP
events on its stream, and the CPU oracle timed on this host's cores; beside it:
  * provider_path: the same layer as the reference's executor issues it through the provider
    table (Gemv QKV, Gemv O, GateUpAct over the stacked gate/up matrix, Gemv down), captured once
    per weight copy and replayed;
  * cfg1 (Q4_0 4096x4096 at one row), cfg2 (Q8_0 14336x4096 at 1, 8, 32 and 128 rows) and
    rows_2_8 (Q4_K at 2, 4 and 8 rows against one row);
  * moe (the MoE layer at 64 decode tokens) and prefill (the 2048-token dense GEMMs on the matrix
    cores and the skewed MoE layer);
  * read_floor: a bare read of each decode op's byte count (the fastest of three read shapes, two of
    them the decode GEMV's own wavefront pattern with no arithmetic), timed like the ops: what one
    launch of that size costs.
--only runs one part (for the profiler); `copy` and `calib` run the counter calibration kernels.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV weight GB/s (% HBM peak); MoE layer tokens/s at 64-token decode"
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
# Non-packed F32 VALU issue: 256 CUs x 4 SIMDs x 16 lanes at the 2.4 GHz peak engine clock, in
# tera lane-operations per second (a wave64 VALU instruction holds a 16-lane SIMD four cycles)
VALU_PEAK_TOPS = 256 * 4 * 16 * 2.4e9 / 1e12
LAYER = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate", 14336, 4096), ("up", 14336, 4096),
         ("down", 4096, 14336)]
Q4K, Q8_0, Q4_0 = 12, 8, 2
SPLIT = 2  # the weight layout of Q8_0 / Q4_0 matrices after repack (codes, then scales)
COPIES = 5
MALL_BYTES = 256 << 20
PARTS = ["layer", "provider", "cfgs", "rows", "floor", "moe", "prefill"]


def q4k_bytes(n_out, k):
    return n_out * (k // 256) * 144


def row_bytes(ty, k):
    return {Q4K: k // 256 * 144, Q8_0: k // 32 * 34, Q4_0: k // 32 * 18}[ty]


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", choices=PARTS + ["copy", "calib"], default=None)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=8.0)
    p.add_argument("--no-moe", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    return p.parse_args()


def S_lib():
    from syntropy_amd._lib import lib
    return lib()


def gpu_us(torch, fn, n):
    """Average GPU time of fn(i) for i < n, launched back to back on the current stream: a spin
    kernel first, so every launch is queued before the GPU reaches it and the event pair times
    the kernels (launch gaps included), not the host's rate."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(4e7))
    e0.record()
    for i in range(n):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e3


def host_info():
    """This host's CPU as lscpu reports it, and the cores this process may use."""
    info = {"cpus_visible": os.cpu_count(), "cpus_in_affinity": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        want = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
                "Thread(s) per core": "threads_per_core", "CPU(s)": "cpus"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in want:
                info[want[k.strip()]] = v.strip()
        flags = next((ln for ln in out.splitlines() if ln.startswith("Flags:")), "")
        info["isa"] = "avx512" if "avx512f" in flags else "avx2" if "avx2" in flags else "baseline"
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def cpu_threads():
    # one GPU's share of the host is 16 threads; no more than the process may use
    return max(1, min(16, len(os.sched_getaffinity(0))))


# ---- the headline: the decode layer ---------------------------------------------------------------
def timed_reps(fn, seconds):
    """(repetitions, seconds) of fn run back to back for at least `seconds` (one call first, untimed)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return n, dt


# The CPU baseline is the reference's own x86 level of kernels-cpu restated in C
# (crates/kernels-cpu/src/gemv/x86.rs: AVX2 block sums, 8 activation rows a weight pass), the
# same bits as the portable restatement, which is timed beside it for a shorter sample.
CPU_LEVEL, PORTABLE_SECONDS = 1, 2.0


def build_layer(torch, S, seed_base):
    gen = torch.Generator(device="cuda")
    copies = []
    for c in range(COPIES):
        mats = {}
        for i, (name, n_out, k) in enumerate(LAYER):
            gen.manual_seed(seed_base + 100 * c + i)
            w = torch.randn(n_out * k, generator=gen, device="cuda", dtype=torch.float32) * 0.02
            mats[name] = S.repack(S.Weights(S.WeightType.Q4K, S.quantize(S.WeightType.Q4K, w), n_out, k))
            del w
        copies.append(mats)
    gen.manual_seed(seed_base + 7)
    xs = {name: torch.randn(k, generator=gen, device="cuda", dtype=torch.float32) for name, _, k in LAYER}
    ys = {name: torch.empty(n_out, device="cuda", dtype=torch.float32) for name, n_out, _ in LAYER}
    wss = {}
    for name, _, k in LAYER:
        need = C.c_uint64()
        S_lib().syn_gemv_layout_workspace_bytes(1, Q4K, 1, k, C.byref(need))
        wss[name] = torch.empty(max(need.value, 256), dtype=torch.uint8, device="cuda")
    return copies, xs, ys, wss


def run_step(S, mats, xs, ys, wss, stream):
    """One decode layer: five Gemv ops (F32 row in, Q8_K quantization fused, F32 row out)."""
    for name, _, _ in LAYER:
        S.gemv(mats[name], xs[name], 1, y=ys[name], ws=wss[name], stream=stream)


def bench_layer(torch, S, a, copies, xs, ys, wss):
    stream = torch.cuda.current_stream()
    names = [name for name, _, _ in LAYER]
    batches = [S.GemvBatch([c[n] for n in names], [xs[n] for n in names], [ys[n] for n in names])
               for c in copies]
    weight_bytes = sum(q4k_bytes(n, k) for _, n, k in LAYER)
    # the layer's five Gemv ops as one grouped launch pair per step (syn_gemv_batch_layout)
    for i in range(a.warmup):
        batches[i % COPIES](stream=stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        batches[i % COPIES](stream=stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    value = weight_bytes * a.steps / dt / 1e9
    # the same five ops launched one by one (one launch each, quantization fused)
    for i in range(a.warmup):
        run_step(S, copies[i % COPIES], xs, ys, wss, stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for i in range(a.steps):
        run_step(S, copies[i % COPIES], xs, ys, wss, stream)
    torch.cuda.synchronize()
    dt_ops = time.perf_counter() - t1
    nrep = max(20, min(a.steps, 100))
    # the grouped GEMV launch (the dominant kernel) alone, back to back on its stream
    for b in batches:
        b.quantize(stream)
    batch_us = gpu_us(torch, lambda i: batches[i % COPIES].gemv_quantized(stream), nrep)
    per = {name: gpu_us(torch, lambda i, name=name: S.gemv(copies[i % COPIES][name], xs[name], 1, y=ys[name],
                                                             ws=wss[name], stream=stream), nrep)
           for name, _, _ in LAYER}
    # algorithmic bytes of one grouped launch: the weights, each Q8_K row once (codes, 32-value
    # sums, scales) and the F32 outputs
    alg_bytes = sum(q4k_bytes(n, k) + k + k // 8 + k // 64 + 4 * n for _, n, k in LAYER)
    achieved = alg_bytes / (batch_us * 1e-6) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_q4k_gemv_decode_layer.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")
    return {
        "value": round(value, 2),
        "ms_per_step": round(dt / a.steps * 1e3, 5),
        "config": {
            "workload": "Q4_K decode layer matmuls, Llama-3-8B shapes, batch 1: QKV 6144x4096, "
                        "O 4096x4096, gate/up 14336x4096, down 4096x14336; Q8_K act quant + "
                        "5 GEMVs per step",
            "launch": "grouped: one batched Q8_K quantization + one grouped GEMV (syn_gemv_batch_layout)",
            "weight_layout": "X8 (runs of 8 Q4_K super-blocks stored chunk-major; repacked once at load)",
            "weight_bytes_per_step": weight_bytes,
            "weight_copies_rotated": COPIES,
            "hbm_fraction_of_peak": round(value / HBM_PEAK_GBS, 4),
            "one_op_per_launch_gbs": round(weight_bytes * a.steps / dt_ops / 1e9, 2),
            "one_op_per_launch_us": {k: round(v, 3) for k, v in per.items()},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_gemv_q4k_batch<X8> (syn_gemv_batch_quantized_layout: the grouped GEMV on Q8_K rows)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/traffic_q4k_gemv_decode_layer.json (rocprofv3 --pmc FETCH_SIZE, "
                              "WRITE_SIZE, scaled by the calibration kernels)",
            "alg_bytes_per_launch": alg_bytes,
            "avg_launch_us": round(batch_us, 3),
        },
    }


def cpu_layer_baseline(copies, xs, seconds):
    """The oracle (C restatement of crates/kernels-cpu, multi-threaded by the reference's row
    partition) over the same layer: a bounded sample of `seconds` of repeated layers, then one
    layer at one thread (a reference launch runs on the calling thread)."""
    from oracle import oracle as o
    threads = cpu_threads()
    mats = copies[0]
    w = {}
    for name, _, _ in LAYER:  # the oracle reads the GGUF order: undo the X8 repack on the host
        b = mats[name].bytes.cpu().numpy()
        src = np.empty_like(b)
        S_lib().syn_q4k_repack_host(1, b.ctypes.data, src.ctypes.data, b.size, 1)
        w[name] = src
    x = {name: xs[name].cpu().numpy() for name, _, _ in LAYER}
    total_w = sum(q4k_bytes(n, k) for _, n, k in LAYER)

    def layer(t, level=CPU_LEVEL):
        for name, n_out, k in LAYER:
            o.gemv(o.Q4_K, w[name], n_out, k, x[name], 1, threads=t, level=level)

    n, dt = timed_reps(lambda: layer(threads), seconds)
    reps1, dt1 = timed_reps(lambda: layer(1), 1.0)
    one = dt1 / reps1
    np_, dtp = timed_reps(lambda: layer(threads, 0), PORTABLE_SECONDS)
    return {
        "value": round(total_w * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "level": "x86 (AVX2 block sums, crates/kernels-cpu/src/gemv/x86.rs)",
        "sample": f"{n} Q4_K decode layers (5 GEMVs incl. Q8_K activation quantization) in {dt:.1f} s on "
                  f"{threads} threads (the host's CPU share for one GPU); one layer at 1 thread: "
                  f"{one * 1e3:.2f} ms = {total_w / one / 1e9:.2f} GB/s",
        "ms_per_layer": round(dt / n * 1e3, 3),
        "one_thread_gbs": round(total_w / one / 1e9, 3),
        "portable_gbs": round(total_w * np_ / dtp / 1e9, 3),
        "host": host_info(),
    }


# ---- the layer through the provider table ----------------------------------------------------------
def bench_provider(torch, S, a, copies, xs):
    """QKV Gemv, O Gemv, GateUpAct{Silu} over the stacked [gate; up] matrix and down Gemv, the
    reference's dense lowering (crates/graph/src/blocks/ffn.rs:39-60), each a prepared op of the
    provider table (X8 weights), captured once per weight copy and replayed."""
    from syntropy_amd import provider as P
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemcpy.restype = C.c_int
    pr = P.Provider()
    ctx = pr.open(0)
    try:
        s = pr.stream(ctx)
        # the stacked [gate; up] matrix: gate holds whole 8-block X8 runs, so its X8 form is the two
        # X8 matrices one after the other
        gateup = [torch.cat([c["gate"].bytes, c["up"].bytes]) for c in copies]
        ops = [("qkv", "Gemv", 6144, 4096), ("o", "Gemv", 4096, 4096), ("gateup", {"GateUpAct": {"act": "Silu"}},
                                                                      14336, 4096), ("down", "Gemv", 4096, 14336)]
        prepared = []
        for name, op, n, k in ops:
            key = {"op": op, "schemes": [{"Ggml": "Q4_K"}, {"Plain": "F32"}, {"Plain": "F32"}], "layout": 1,
                   "variant": 0}
            po = pr.prepare(ctx, key, {"class": "Decode", "rows": 1, "dims": [n, k]})
            xb, yb, ws = pr.alloc(ctx, 4 * k), pr.alloc(ctx, 4 * n), pr.alloc(ctx, po.workspace)
            xh = xs["gate" if name == "gateup" else name].cpu().numpy()
            assert hip.hipMemcpy(xb.addr, xh.ctypes.data, xh.nbytes, 1) == 0
            per_copy = []
            for c in range(COPIES):
                wt = gateup[c] if name == "gateup" else copies[c][name].bytes
                per_copy.append(P.op_args([P.packed(xb, P.DT_F32, [1, k])], [P.packed(yb, P.DT_F32, [1, n])],
                                          [P.view(wt.data_ptr(), wt.numel())], P.Slice(ws.handle, 0, po.workspace)))
            prepared.append((name, po, per_copy))
        weight_bytes = sum(q4k_bytes(n * (2 if nm == "gateup" else 1), k) for nm, _, n, k in ops)
        e0, e1 = pr.event(ctx), pr.event(ctx)

        def graphs_of(names):
            gs = []
            for c in range(COPIES):
                pr.begin_capture(ctx, s)
                for name, po, per_copy in prepared:
                    if name in names:
                        pr.launch(ctx, s, po, per_copy[c])
                gs.append(pr.end_capture(ctx, s))
            for g in gs:
                pr.replay(ctx, s, g)
            pr.synchronize(ctx, s)
            return gs

        def replay_us(gs, n):
            pr.synchronize(ctx, s)
            pr.record(ctx, s, e0)
            for i in range(n):
                pr.replay(ctx, s, gs[i % COPIES])
            pr.record(ctx, s, e1)
            pr.synchronize(ctx, s)
            return pr.elapsed(ctx, e0, e1) / n / 1e3

        layer_graphs = graphs_of([nm for nm, _, _, _ in ops])
        step_us = replay_us(layer_graphs, a.steps)
        per_op = {nm: round(replay_us(graphs_of([nm]), max(20, a.steps // 2)), 3) for nm, _, _, _ in ops}
        gbs = weight_bytes / (step_us * 1e-6) / 1e9
        return {
            "workload": "the decode layer through the provider table: Gemv QKV 6144x4096, Gemv O "
                        "4096x4096, GateUpAct{Silu} 2x14336x4096 (stacked gate/up), Gemv down 4096x14336; "
                        "X8 weights; one captured graph per weight copy, replayed",
            "weight_bytes_per_step": weight_bytes,
            "us_per_step": round(step_us, 3),
            "gbs": round(gbs, 1),
            "hbm_fraction_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "per_op_graph_us": per_op,
            "per_op_gbs": {nm: round(q4k_bytes(n * (2 if nm == "gateup" else 1), k) / (per_op[nm] * 1e-6) / 1e9, 1)
                           for nm, _, n, k in ops},
        }
    finally:
        pr.close(ctx)


# ---- Cfg1, Cfg2 and rows 2-8 ------------------------------------------------------------------------
def weight_set(torch, S, ty, n, k, seed, layout=0):
    """Copies of one N(0, 0.02) matrix quantized by the GPU packer, enough to exceed the MALL."""
    wty = {Q4K: S.WeightType.Q4K, Q8_0: S.WeightType.Q8_0, Q4_0: S.WeightType.Q4_0}[ty]
    ncopies = max(COPIES, -(-2 * MALL_BYTES // (n * row_bytes(ty, k))))
    gen = torch.Generator(device="cuda")
    out = []
    for c in range(ncopies):
        gen.manual_seed(seed + c)
        w = torch.randn(n * k, generator=gen, device="cuda") * 0.02
        W = S.Weights(wty, S.quantize(wty, w), n, k)
        out.append(S.repack(W) if layout else W)
    return out


def gemv_case(torch, S, ws_list, rows, n, k, nrep, kernel=True):
    """(step us: quantization + GEMV, kernel us: the GEMV on quantized rows, or None when not
    asked for) at `rows` rows."""
    ty = ws_list[0].ty
    x = torch.randn(rows, k, device="cuda")
    y = torch.empty(rows, n, device="cuda")
    lay = ws_list[0].layout
    need = C.c_uint64()
    S_lib().syn_gemv_layout_workspace_bytes(lay, int(ty), rows, k, C.byref(need))
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device="cuda")
    step = gpu_us(torch, lambda i: S.gemv(ws_list[i % len(ws_list)], x, rows, y=y, ws=ws), nrep)
    kern = None
    if kernel and lay in (0, 2):  # the product alone, over rows quantized beforehand
        qws = S.new_workspace(ty, rows, k)
        S.quantize_into(ty, x, rows, k, qws)
        kern = gpu_us(torch, lambda i: S.gemv_quantized(ws_list[i % len(ws_list)], qws, rows, y), nrep)
    return step, kern


def bench_cfgs(torch, S, a):
    nrep = max(20, min(a.steps, 100))
    res = {}
    # Cfg1: Q4_0 4096 x 4096 at one row
    n, k = 4096, 4096
    wl = weight_set(torch, S, Q4_0, n, k, 0x51A10001, SPLIT)
    step, kern = gemv_case(torch, S, wl, 1, n, k, nrep)
    wb = n * row_bytes(Q4_0, k)
    alg = wb + 4 * k + 4 * n  # the op is one launch: weights, the F32 row, the outputs
    res["cfg1"] = {"workload": "Q4_0 4096x4096 Gemv, one F32 row (quantized to Q8_0 blocks inside the GEMV's "
                               "workgroups: one launch), weights in the SPLIT layout",
                   "weight_bytes": wb, "copies_rotated": len(wl), "step_us": round(step, 3),
                   "weight_gbs": round(wb / (step * 1e-6) / 1e9, 1),
                   "product_on_a_quantized_row_us": round(kern, 3),
                   "roofline": {"bound": "hbm", "kernel": "k_gemv_split<Q4_0,1,2> (row quantized in the workgroups)",
                                "achieved": round(alg / (step * 1e-6) / 1e9, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(alg / (step * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                "alg_bytes_per_launch": alg, "avg_launch_us": round(step, 3)}}
    del wl
    # Cfg2: Q8_0 14336 x 4096 at 1, 8, 32 and 128 rows
    n, k = 14336, 4096
    wl = weight_set(torch, S, Q8_0, n, k, 0x51A10002, SPLIT)
    wb = n * row_bytes(Q8_0, k)
    rows_res = {}
    for T in (1, 8, 32, 128):
        step, kern = gemv_case(torch, S, wl, T, n, k, max(10, nrep // (1 + T // 32)))
        if T == 1:  # one launch: the row quantized in the product's workgroups
            alg, kt = wb + 4 * k + 4 * n, step
        else:
            alg, kt = wb + T * (k + 8 * (k // 32)) + 4 * T * n, kern
        rows_res[str(T)] = {"kernel": "k_gemv_split<Q8_0,1,2> (row quantized in the workgroups)" if T == 1
                            else "k_gemm_q8_staged",
                            "step_us": round(step, 3), "weight_gbs": round(wb / (step * 1e-6) / 1e9, 1),
                            "kernel_us": round(kt, 3), "kernel_alg_gbs": round(alg / (kt * 1e-6) / 1e9, 1),
                            "kernel_frac": round(alg / (kt * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                            "tflops": round(2.0 * T * n * k / (step * 1e-6) / 1e12, 2)}
        if T > 1:
            # the F32 term of every (output, block): convert, two multiplies, add (gemv.rs:539-547),
            # one VALU lane-operation each, against the VALU issue peak
            ops = 4.0 * T * n * (k // 32)
            rows_res[str(T)]["valu_roofline"] = {
                "bound": "valu", "ops_per_launch": int(ops), "unit": "T lane-ops/s",
                "achieved": round(ops / (kt * 1e-6) / 1e12, 2), "peak": round(VALU_PEAK_TOPS, 2),
                "frac": round(ops / (kt * 1e-6) / 1e12 / VALU_PEAK_TOPS, 4)}
        if T == 1:
            rows_res["1"]["product_on_a_quantized_row_us"] = round(kern, 3)
    res["cfg2"] = {"workload": "Q8_0 14336x4096 (Llama-3-8B FFN up) Gemv at T rows, Q8_0 activations, "
                               "weights in the SPLIT layout",
                   "weight_bytes": wb, "copies_rotated": len(wl), "rows": rows_res}
    del wl
    torch.cuda.empty_cache()
    return res


def bench_rows(torch, S, a):
    """RFC-0040 9 row 2: rows 2-8 at most 1.10 x the one-row time (Q4_K 14336x4096, both layouts)."""
    nrep = max(20, min(a.steps, 100))
    n, k = 14336, 4096
    out = {"target": "time(rows) <= 1.10 x time(rows = 1) (RFC-0040 9, row 2)", "shape": [n, k]}
    for layout in (0, 1):
        wl = weight_set(torch, S, Q4K, n, k, 0x51A10004, layout)
        t = {}
        for rows in (1, 2, 4, 8):
            t[rows], _ = gemv_case(torch, S, wl, rows, n, k, nrep, kernel=False)
        out["x8" if layout else "source"] = {"us": {str(r): round(v, 3) for r, v in t.items()},
                                             "ratio": {str(r): round(t[r] / t[1], 3) for r in (2, 4, 8)}}
        del wl
        torch.cuda.empty_cache()
    return out


# ---- MoE at 64 decode tokens ------------------------------------------------------------------------
MOE = dict(n_experts=128, top_k=8, hidden=4096, inter=1536, tokens=64)


def build_moe(torch, S, M, seed):
    """Qwen3-235B-A22B MoE layer shape: router F32 N(0,0.02); 128 experts of gate/up [1536,4096]
    and down [4096,1536], N(0,0.02) quantized to Q4_K by the GPU packer; x N(0,1)."""
    c = MOE
    gen = torch.Generator(device="cuda")
    mats = []
    for m, (n_out, k) in enumerate([(c["inter"], c["hidden"]), (c["inter"], c["hidden"]),
                                    (c["hidden"], c["inter"])]):
        parts = []
        for e in range(c["n_experts"]):
            gen.manual_seed(seed + 1000 * m + e)
            w = torch.randn(n_out * k, generator=gen, device="cuda", dtype=torch.float32) * 0.02
            parts.append(S.quantize(S.WeightType.Q4K, w))
        mats.append(torch.cat(parts))
        del parts
    gen.manual_seed(seed + 7)
    router = torch.randn(c["n_experts"], c["hidden"], generator=gen, device="cuda") * 0.02
    x = torch.randn(c["tokens"], c["hidden"], generator=gen, device="cuda")
    shape = M.MoeShape(c["n_experts"], c["top_k"], c["hidden"], c["inter"])
    layer = M.MoeLayer(shape, router, M.Experts(12, *mats), c["tokens"])
    return layer, x


def bench_moe(torch, S, M, steps, warmup, cpu_seconds):
    c = MOE
    layer, x = build_moe(torch, S, M, 0x51A40000)
    gguf = layer.experts

    def timed(experts):
        layer.experts = experts
        for _ in range(warmup):
            layer(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            r = layer(x)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, r

    # the experts repacked once at load (TILE64: each 64-row run stored super-block-major), and
    # the same layer over the GGUF-order experts, in alternating rounds (the median of each)
    tiled = M.tile64(gguf, layer.s)
    rounds = [(timed(tiled), timed(gguf)) for _ in range(5)]
    dt = sorted(r[0][0] for r in rounds)[2]
    dt_src = sorted(r[1][0] for r in rounds)[2]
    y, ids, w, out = rounds[-1][0][1]
    y_src = rounds[-1][1][1][0]
    layer.experts = gguf
    if not torch.equal(y.view(torch.int32), y_src.view(torch.int32)):
        raise SystemExit("bench: the MoE layer differs between the expert layouts")
    ids_h = ids.cpu().numpy()
    e_t = len(set(ids_h.ravel().tolist()))
    loads = [int((ids_h == e).sum()) for e in range(c["n_experts"])]
    expert_bytes = 3 * c["inter"] * (c["hidden"] // 256) * 144
    alg = e_t * expert_bytes + c["n_experts"] * c["hidden"] * 4 + 2 * c["tokens"] * c["hidden"] * 4
    ms = dt / steps * 1e3
    res = {
        "metric": "MoE layer tokens/s at 64-token decode",
        "value": round(c["tokens"] * steps / dt, 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms, 4),
        "workload": "Qwen3-235B-A22B MoE FFN shape: 64 decode tokens, hidden 4096, 128 Q4_K experts "
                    "(SwiGLU inter 1536), softmax top-8 renormalized; route + pack + grouped FFN + combine",
        "expert_layout": "TILE64 (repacked once at load)",
        "timing": f"median of 5 rounds of {steps} steps, alternating with the GGUF-order experts",
        "ms_per_step_gguf_layout": round(dt_src / steps * 1e3, 4),
        "distinct_experts": e_t,
        "max_over_avg_load": round(max(loads) / (sum(loads) / c["n_experts"]), 3),
        "alg_bytes_per_step": alg,
        "hbm_gbs": round(alg / (ms * 1e-3) / 1e9, 1),
        "hbm_fraction_of_peak": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    if cpu_seconds > 0:
        from oracle import oracle as o
        threads = cpu_threads()
        ex = layer.experts
        g, u, d = ex.gate.cpu().numpy(), ex.up.cpu().numpy(), ex.down.cpu().numpy()
        r, xh = layer.router.cpu().numpy(), x.cpu().numpy()

        def step(level=CPU_LEVEL):
            ids_c, w_c, _ = o.moe_route(r, xh, c["n_experts"], c["top_k"], True)
            out_c = o.moe_grouped(o.Q4_K, o.Q4_K, c["n_experts"], c["top_k"], c["hidden"],
                                  c["inter"], g, u, d, xh, ids_c, threads=threads, level=level)
            return o.moe_combine_ranked(out_c, w_c)

        n, cdt = timed_reps(step, cpu_seconds)
        np_, dtp = timed_reps(lambda: step(0), PORTABLE_SECONDS)
        res["cpu_baseline"] = {"value": round(c["tokens"] * n / cdt, 1), "unit": "tokens/s",
                               "cores": threads, "kind": "port",
                               "level": "x86 (AVX2 block sums, crates/kernels-cpu/src/gemv/x86.rs)",
                               "sample": f"{n} MoE layers of 64 tokens in {cdt:.1f} s (experts split over "
                                         f"{threads} threads)",
                               "portable_tokens_per_s": round(c["tokens"] * np_ / dtp, 1)}
        res["speedup_over_cpu"] = round(res["value"] / res["cpu_baseline"]["value"], 1)
    return res


# ---- prefill at 2048 tokens ---------------------------------------------------------------------------
PREFILL = dict(tokens=2048, dense=[("gate", 14336, 4096), ("down", 4096, 14336)], skew_rows=(3, 50, 97),
               skew_scale=3.0)


def bench_prefill(torch, S, M, steps, warmup, cpu_seconds):
    """Prefill at 2048 tokens: the dense Q4_K GEMMs (2048x4096 activations, BF16-valued, times
    gate 14336x4096 and down 4096x14336) on the matrix cores, and the MoE layer at 2048 tokens
    with three router rows scaled so their experts take several times the average load."""
    c = PREFILL
    T = c["tokens"]
    gen = torch.Generator(device="cuda")
    mats, xs, wss, ys = {}, {}, {}, {}
    for i, (name, n_out, k) in enumerate(c["dense"]):
        gen.manual_seed(0x51A10005 + i)
        w = torch.randn(n_out * k, generator=gen, device="cuda") * 0.02
        mats[name] = S.Weights(S.WeightType.Q4K, S.quantize(S.WeightType.Q4K, w), n_out, k)
        del w
        gen.manual_seed(0x51A20005 + i)
        xs[name] = torch.randn(T, k, generator=gen, device="cuda").to(torch.bfloat16).float()
        wss[name] = S.gemm_workspace(T, k)
        ys[name] = torch.empty(T, n_out, device="cuda")
    stream = torch.cuda.current_stream()

    def dense_step():
        for name, _, k in c["dense"]:
            S.gemm_quantize_into(xs[name], T, k, wss[name], stream=stream)
            S.gemm_quantized(mats[name], wss[name], T, ys[name], stream=stream)

    for _ in range(warmup):
        dense_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dense_step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    flops = sum(2.0 * T * n * k for _, n, k in c["dense"])
    per = {}
    for name, _, k in c["dense"]:  # the GEMM kernel alone, HIP events on its stream
        S.gemm_quantize_into(xs[name], T, k, wss[name], stream=stream)
        per[name] = gpu_us(torch, lambda i, name=name: S.gemm_quantized(mats[name], wss[name], T, ys[name],
                                                                        stream=stream), steps)
    gemm_s = sum(per.values()) * 1e-6
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_prefill_gemm_2048tok.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")
    res = {
        "workload": "prefill, 2048 tokens: X 2048x4096 (BF16 values) x Q4_K gate 14336x4096, "
                    "X' 2048x14336 x Q4_K down 4096x14336; Q8_K activation quantization + GEMM each",
        "dense_tokens_per_s": round(T / dt, 1),
        "dense_ms_per_step": round(dt * 1e3, 4),
        "dense_tflops": round(flops / dt / 1e12, 1),
        "roofline": {"bound": "mfma", "kernel": "k_gemm_q4k (F16 MFMA, exact integer sums)",
                     "achieved": round(flops / gemm_s / 1e12, 1), "peak": F16_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / gemm_s / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_source": "profiles/traffic_prefill_gemm_2048tok.json (rocprofv3 --pmc)",
                     "avg_launch_us": {k: round(v, 1) for k, v in per.items()}},
    }
    del mats, xs, wss, ys
    torch.cuda.empty_cache()
    mc = MOE
    layer, _ = build_moe(torch, S, M, 0x51A40000)
    router = layer.router.clone()
    for r in c["skew_rows"]:
        router[r] *= c["skew_scale"]
    gen.manual_seed(0x51A20006)
    x = torch.randn(T, mc["hidden"], generator=gen, device="cuda")
    gguf = layer.experts
    big = M.MoeLayer(layer.s, router, gguf, T)

    def timed(experts):
        big.experts = experts
        for _ in range(max(1, warmup // 2)):
            big(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            r = big(x)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, r

    # the experts repacked to TILE64 once at load, as the decode layer's; the GGUF order beside
    # them, in alternating rounds (the median of each)
    tiled = M.tile64(gguf, layer.s)
    rounds = [(timed(tiled), timed(gguf)) for _ in range(3)]
    mdt = sorted(r[0][0] for r in rounds)[1]
    mdt_src = sorted(r[1][0] for r in rounds)[1]
    y, ids, w, out = rounds[-1][0][1]
    if not torch.equal(y.view(torch.int32), rounds[-1][1][1][0].view(torch.int32)):
        raise SystemExit("bench: the 2048-token MoE layer differs between the expert layouts")
    big.experts = gguf
    ids_h = ids.cpu().numpy()
    loads = sorted((int((ids_h == e).sum()) for e in range(mc["n_experts"])), reverse=True)
    avg = T * mc["top_k"] / mc["n_experts"]
    moe_flops = 2.0 * T * mc["top_k"] * 3 * mc["inter"] * mc["hidden"]
    res["moe"] = {"tokens_per_s": round(T / mdt, 1), "ms_per_step": round(mdt * 1e3, 3),
                  "tflops": round(moe_flops / mdt / 1e12, 1),
                  "expert_layout": "TILE64 (repacked once at load)",
                  "ms_per_step_gguf_layout": round(mdt_src * 1e3, 3),
                  "top_loads_over_avg": [round(v / avg, 2) for v in loads[:4]],
                  "skew": f"router rows {list(c['skew_rows'])} scaled by {c['skew_scale']}"}
    if cpu_seconds > 0:
        from oracle import oracle as o
        threads = cpu_threads()
        rows = 16
        sample = []
        for i, (name, n_out, k) in enumerate(c["dense"]):
            gen.manual_seed(0x51A10005 + i)
            w = torch.randn(n_out * k, generator=gen, device="cuda") * 0.02
            wb = S.quantize(S.WeightType.Q4K, w).cpu().numpy()
            xh = torch.randn(rows, k, device="cuda").cpu().numpy()
            sample.append((wb, n_out, k, xh))
        def dense(level=CPU_LEVEL):
            for wb, n_out, k, xh in sample:
                o.gemv(o.Q4_K, wb, n_out, k, xh, rows, threads=threads, level=level)

        n, cdt = timed_reps(dense, cpu_seconds)
        np_, dtp = timed_reps(lambda: dense(0), PORTABLE_SECONDS)
        res["cpu_baseline"] = {"value": round(rows * n / cdt, 1), "unit": "tokens/s (dense gate+down)",
                               "cores": threads, "kind": "port",
                               "level": "x86 (AVX2 block sums, 8 rows a weight pass, "
                                        "crates/kernels-cpu/src/gemv/x86.rs, gemv.rs:83)",
                               "sample": f"{n} x {rows} token rows through gate and down in {cdt:.1f} s",
                               "portable_tokens_per_s": round(rows * np_ / dtp, 1)}
        res["speedup_over_cpu"] = round(res["dense_tokens_per_s"] / res["cpu_baseline"]["value"], 1)
    return res


# ---- counter calibration kernels --------------------------------------------------------------------
def bench_read_floor(torch, nrep):
    """A bare read of each decode op's weight bytes, launched back to back over copies that
    together exceed the Infinity Cache, in three shapes: syn_hbm_read_probe (one 16-byte load a
    lane, 4 KB a workgroup) and syn_hbm_read_runs at 1 and 8 wavefronts a workgroup (the X8 decode
    GEMV's own wavefront pattern, 9 KB a wavefront).  The fastest is the time one launch of that
    many bytes takes with no arithmetic, against which an op's time is measured."""
    f = S_lib().syn_hbm_read_probe_sink_words
    f.argtypes, f.restype = [C.c_uint64], C.c_uint64
    g = S_lib().syn_hbm_read_runs_sink_words
    g.argtypes, g.restype = [C.c_uint64], C.c_uint64
    sizes = {"O 4096x4096 Q4_K / Cfg1 Q4_0 4096x4096": 4096 * row_bytes(Q4K, 4096),
             "QKV 6144x4096 Q4_K": 6144 * row_bytes(Q4K, 4096),
             "gate, up or down Q4_K": 14336 * row_bytes(Q4K, 4096),
             "Cfg2 Q8_0 14336x4096": 14336 * row_bytes(Q8_0, 4096),
             "decode layer Q4_K (5 GEMVs)": 122683392,
             "512 MiB": 512 << 20}
    out = {}
    stream = torch.cuda.current_stream().cuda_stream
    for name, nbytes in sizes.items():
        nbytes = nbytes // 16 * 16
        ncopies = max(3, -(-2 * MALL_BYTES // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(c) for c in range(ncopies)]
        sink = torch.empty(max(f(nbytes), g(nbytes)), dtype=torch.int32, device="cuda")
        shapes = {}
        for shape in ("probe", "runs1", "runs8"):
            def go(i, shape=shape):
                src = bufs[i % ncopies].data_ptr()
                if shape == "probe":
                    rc = S_lib().syn_hbm_read_probe(src, nbytes, sink.data_ptr(), stream)
                else:
                    rc = S_lib().syn_hbm_read_runs(1 if shape == "runs1" else 8, src, nbytes, sink.data_ptr(), stream)
                assert rc == 0
            go(0)
            shapes[shape] = round(gpu_us(torch, go, nrep), 3)
        best = min(shapes, key=shapes.get)
        us = shapes[best]
        out[name] = {"bytes": nbytes, "us": us, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "shape": best,
                     "us_by_shape": shapes}
        del bufs, sink
    torch.cuda.empty_cache()
    return out


def calibrate(torch, only):
    """`copy`: a plain 512 MiB device copy (reads and writes 512 MiB each); `calib`: 512 MiB read
    once by syn_hbm_read_probe with the decode GEMV's load pattern.  Five launches each."""
    nbytes = 512 << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    if only == "copy":
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        written = nbytes
    else:
        f = S_lib().syn_hbm_read_probe_sink_words
        f.argtypes, f.restype = [C.c_uint64], C.c_uint64
        words = f(nbytes)
        sink = torch.empty(words, dtype=torch.int32, device="cuda")
        for _ in range(5):
            rc = S_lib().syn_hbm_read_probe(src.data_ptr(), nbytes, sink.data_ptr(),
                                            torch.cuda.current_stream().cuda_stream)
            assert rc == 0
        written = 4 * words
    torch.cuda.synchronize()
    print(json.dumps({"kernel": only, "bytes_read_per_launch": nbytes, "bytes_written_per_launch": written,
                      "launches": 5}))


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {a.gpus} is not supported (one GPU only)", file=sys.stderr)
        sys.exit(2)
    import torch
    import syntropy_amd.gemv as S
    import syntropy_amd.moe as M

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    torch.cuda.set_device(0)
    if a.only in ("copy", "calib"):
        calibrate(torch, a.only)
        return
    want = set(PARTS) if a.only is None else {a.only}
    if a.no_moe:
        want.discard("moe")
    if a.no_prefill:
        want.discard("prefill")
    out = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "i8xi8->i32, f32 terms",
           "data": "synthetic: W ~ N(0,0.02) -> Q4_K (GPU packer, ggml-exact); x ~ N(0,1) F32"}
    if want & {"layer", "provider"}:
        copies, xs, ys, wss = build_layer(torch, S, 0x51A10003)
        if "layer" in want:
            lay = bench_layer(torch, S, a, copies, xs, ys, wss)
            out["value"], out["ms_per_step"] = lay["value"], lay["ms_per_step"]
            out["config"], out["roofline"] = lay["config"], lay["roofline"]
            if not a.no_cpu:
                out["cpu_baseline"] = cpu_layer_baseline(copies, xs, a.cpu_seconds)
                # the whole GPU step (quantization + GEMVs) against the CPU path's whole layer
                out["speedup_over_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
        if "provider" in want:
            out["provider_path"] = bench_provider(torch, S, a, copies, xs)
        del copies, xs, ys, wss
        torch.cuda.empty_cache()
    if "cfgs" in want:
        out.update(bench_cfgs(torch, S, a))
    if "rows" in want:
        out["rows_2_8"] = bench_rows(torch, S, a)
    if "floor" in want:
        out["read_floor"] = bench_read_floor(torch, max(20, min(a.steps, 100)))
    if "moe" in want:
        torch.cuda.empty_cache()
        out["moe"] = bench_moe(torch, S, M, max(10, a.steps // 4), max(3, a.warmup // 4),
                               0 if a.no_cpu else a.cpu_seconds)
    if "prefill" in want:
        torch.cuda.empty_cache()
        out["prefill"] = bench_prefill(torch, S, M, max(5, a.steps // 20), max(2, a.warmup // 10),
                                       0 if a.no_cpu else min(a.cpu_seconds, 5.0))
    print(json.dumps(out))


if __name__ == "__main__":
    main()
