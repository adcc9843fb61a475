#!/usr/bin/env python3
"""Benchmark of the quantized-matmul path on one MI355X.

Headline workload: one Q4_K decode layer's matmuls at Llama-3-8B shapes, batch 1 (QKV
6144x4096, O 4096x4096, gate and up 14336x4096, down 4096x14336).  One step quantizes each
GEMV's F32 activation row to Q8_K and runs the five GEMVs: the reference's `Gemv` op five
times.  Weights are N(0, 0.02) quantized by the GPU Q4_K packer (byte-identical to ggml's),
then repacked once to the X8 layout (the provider's repack: a permutation of the bytes), in
COPIES distinct copies that the steps rotate through, so the weights come from HBM and not
from the 256 MB Infinity Cache.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only layer|copy] [--no-cpu]

Prints one JSON line: whole-step weight GB/s (value), the roofline of the GEMV kernel from
HIP events on its stream, and the CPU oracle timed on this host's cores; beside it the MoE layer
at 64 decode tokens ("moe") and the 2048-token prefill ("prefill": the dense GEMMs on the matrix
cores and the skewed MoE layer).
"""
from __future__ import annotations

import argparse
import json

import numpy as np
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV weight GB/s (% HBM peak); MoE layer tokens/s at 64-token decode"
HBM_PEAK_GBS = 8000.0
LAYER = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate", 14336, 4096), ("up", 14336, 4096),
         ("down", 4096, 14336)]
Q4K = 12
COPIES = 5


def q4k_bytes(n_out, k):
    return n_out * (k // 256) * 144


def act_bytes(k):
    # Q8_K codes + one F32 scale per 256 + one I32 sum per 32, read by the GEMV
    return k + 4 * (k // 256) + 4 * (k // 32)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", choices=["layer", "copy"], default=None)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=8.0)
    p.add_argument("--no-moe", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    return p.parse_args()


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
    xs = {name: torch.randn(k, generator=gen, device="cuda", dtype=torch.float32)
          for name, _, k in LAYER}
    ys = {name: torch.empty(n_out, device="cuda", dtype=torch.float32) for name, n_out, _ in LAYER}
    import ctypes as C
    wss = {}
    for name, _, k in LAYER:
        need = C.c_uint64()
        S_lib().syn_gemv_layout_workspace_bytes(1, Q4K, 1, k, C.byref(need))
        wss[name] = torch.empty(max(need.value, 256), dtype=torch.uint8, device="cuda")
    return copies, xs, ys, wss


def run_step_batched(batch, stream):
    """One decode layer as one grouped launch pair (batched Q8_K quantization + grouped GEMV)."""
    batch(stream=stream)


def run_step(S, mats, xs, ys, wss, stream, events=None):
    """One decode layer: five Gemv ops (F32 row in, Q8_K quantization fused, F32 row out)."""
    for name, _, k in LAYER:
        if events is not None:
            events[name][0].record()
        S.gemv(mats[name], xs[name], 1, y=ys[name], ws=wss[name], stream=stream)
        if events is not None:
            events[name][1].record()


def S_lib():
    from syntropy_amd._lib import lib
    return lib()


def cpu_baseline(torch, copies, xs, seconds):
    """The oracle (C restatement of crates/kernels-cpu, multi-threaded by the reference's row
    partition) over the same layer: bounded sample of `seconds` of repeated layers."""
    from oracle import oracle as o
    threads = min(16, os.cpu_count() or 1)
    mats = copies[0]
    # the oracle reads the GGUF order: undo the X8 repack on the host
    w = {}
    for name, _, _ in LAYER:
        b = mats[name].bytes.cpu().numpy()
        src = np.empty_like(b)
        S_lib().syn_q4k_repack_host(1, b.ctypes.data, src.ctypes.data, b.size, 1)
        w[name] = src
    x = {name: xs[name].cpu().numpy() for name, _, _ in LAYER}
    total_w = sum(q4k_bytes(n, k) for _, n, k in LAYER)

    def layer():
        for name, n_out, k in LAYER:
            o.gemv(o.Q4_K, w[name], n_out, k, x[name], 1, threads=threads)

    layer()
    n, t0 = 0, time.perf_counter()
    while True:
        layer()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    t1 = time.perf_counter()
    layer_single = None
    for name, n_out, k in LAYER:  # one pass at one thread, for reference
        o.gemv(o.Q4_K, w[name], n_out, k, x[name], 1, threads=1)
    layer_single = time.perf_counter() - t1
    return {
        "value": round(total_w * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} Q4_K decode layers (5 GEMVs incl. Q8_K activation quantization) in "
                  f"{dt:.1f} s on {threads} threads; one layer at 1 thread: "
                  f"{layer_single * 1e3:.1f} ms",
        "ms_per_layer": round(dt / n * 1e3, 3),
    }


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
    for _ in range(warmup):
        layer(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        y, ids, w, out = layer(x)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
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
        "distinct_experts": e_t,
        "max_over_avg_load": round(max(loads) / (sum(loads) / c["n_experts"]), 3),
        "alg_bytes_per_step": alg,
        "hbm_gbs": round(alg / (ms * 1e-3) / 1e9, 1),
        "hbm_fraction_of_peak": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    if cpu_seconds > 0:
        from oracle import oracle as o
        threads = min(16, os.cpu_count() or 1)
        ex = layer.experts
        g, u, d = ex.gate.cpu().numpy(), ex.up.cpu().numpy(), ex.down.cpu().numpy()
        r, xh = layer.router.cpu().numpy(), x.cpu().numpy()

        def step():
            ids_c, w_c, _ = o.moe_route(r, xh, c["n_experts"], c["top_k"], True)
            out_c = o.moe_grouped(o.Q4_K, o.Q4_K, c["n_experts"], c["top_k"], c["hidden"],
                                  c["inter"], g, u, d, xh, ids_c, threads=threads)
            return o.moe_combine(out_c, ids_c, w_c)

        step()
        n, t1 = 0, time.perf_counter()
        while True:
            step()
            n += 1
            if time.perf_counter() - t1 >= cpu_seconds:
                break
        cdt = time.perf_counter() - t1
        res["cpu_baseline"] = {"value": round(c["tokens"] * n / cdt, 1), "unit": "tokens/s",
                               "cores": threads, "kind": "port",
                               "sample": f"{n} MoE layers of 64 tokens in {cdt:.1f} s"}
    return res


PREFILL = dict(tokens=2048, dense=[("gate", 14336, 4096), ("down", 4096, 14336)], skew_rows=(3, 50, 97),
               skew_scale=3.0)
F16_MFMA_PEAK_TFLOPS = 2500.0


def bench_prefill(torch, S, M, steps, warmup, cpu_seconds, moe_layer_parts=None):
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
    # the GEMM kernel alone, HIP events on its stream
    per = {}
    for name, _, k in c["dense"]:
        S.gemm_quantize_into(xs[name], T, k, wss[name], stream=stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            S.gemm_quantized(mats[name], wss[name], T, ys[name], stream=stream)
        e1.record()
        torch.cuda.synchronize()
        per[name] = e0.elapsed_time(e1) / steps  # ms
    gemm_s = sum(per.values()) * 1e-3
    res = {
        "workload": "prefill, 2048 tokens: X 2048x4096 (BF16 values) x Q4_K gate 14336x4096, "
                    "X' 2048x14336 x Q4_K down 4096x14336; Q8_K activation quantization + GEMM each",
        "dense_tokens_per_s": round(T / dt, 1),
        "dense_ms_per_step": round(dt * 1e3, 4),
        "dense_tflops": round(flops / dt / 1e12, 1),
        "roofline": {"bound": "mfma", "kernel": "k_gemm_q4k (F16 MFMA, exact integer sums)",
                     "achieved": round(flops / gemm_s / 1e12, 1), "peak": F16_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / gemm_s / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": None, "avg_launch_us": {k: round(v * 1e3, 1) for k, v in per.items()}},
    }
    del mats, xs, wss, ys
    torch.cuda.empty_cache()
    # MoE at 2048 tokens, skewed
    mc = MOE
    layer, _ = build_moe(torch, S, M, 0x51A40000) if moe_layer_parts is None else moe_layer_parts
    router = layer.router.clone()
    for r in c["skew_rows"]:
        router[r] *= c["skew_scale"]
    gen.manual_seed(0x51A20006)
    x = torch.randn(T, mc["hidden"], generator=gen, device="cuda")
    big = M.MoeLayer(layer.s, router, layer.experts, T)
    for _ in range(max(1, warmup // 2)):
        big(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        y, ids, w, out = big(x)
    torch.cuda.synchronize()
    mdt = (time.perf_counter() - t0) / steps
    ids_h = ids.cpu().numpy()
    loads = sorted((int((ids_h == e).sum()) for e in range(mc["n_experts"])), reverse=True)
    avg = T * mc["top_k"] / mc["n_experts"]
    moe_flops = 2.0 * T * mc["top_k"] * 3 * mc["inter"] * mc["hidden"]
    res["moe"] = {"tokens_per_s": round(T / mdt, 1), "ms_per_step": round(mdt * 1e3, 3),
                  "tflops": round(moe_flops / mdt / 1e12, 1),
                  "top_loads_over_avg": [round(v / avg, 2) for v in loads[:4]],
                  "skew": f"router rows {list(c['skew_rows'])} scaled by {c['skew_scale']}"}
    if cpu_seconds > 0:
        from oracle import oracle as o
        threads = min(16, os.cpu_count() or 1)
        rows = 16
        gen.manual_seed(0x51A10005)
        sample = []
        for i, (name, n_out, k) in enumerate(c["dense"]):
            gen.manual_seed(0x51A10005 + i)
            w = torch.randn(n_out * k, generator=gen, device="cuda") * 0.02
            wb = S.quantize(S.WeightType.Q4K, w).cpu().numpy()
            xh = torch.randn(rows, k, device="cuda").cpu().numpy()
            sample.append((wb, n_out, k, xh))
        n, t1 = 0, time.perf_counter()
        while True:
            for wb, n_out, k, xh in sample:
                o.gemv(o.Q4_K, wb, n_out, k, xh, rows, threads=threads)
            n += 1
            if time.perf_counter() - t1 >= cpu_seconds:
                break
        cdt = time.perf_counter() - t1
        res["cpu_baseline"] = {"value": round(rows * n / cdt, 1), "unit": "tokens/s (dense gate+down)",
                               "cores": threads, "kind": "port",
                               "sample": f"{n} x {rows} token rows through gate and down in {cdt:.1f} s"}
    return res


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {a.gpus} is not supported "
              "(one GPU only)", file=sys.stderr)
        sys.exit(2)
    import torch
    import syntropy_amd.gemv as S
    import syntropy_amd.moe as M

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()

    if a.only == "copy":
        # a plain copy of known size: calibrates the HBM byte counters
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel(), "launches": 5}))
        return

    copies, xs, ys, wss = build_layer(torch, S, 0x51A10003)
    names = [name for name, _, _ in LAYER]
    batches = [S.GemvBatch([c[n] for n in names], [xs[n] for n in names], [ys[n] for n in names])
               for c in copies]
    weight_bytes = sum(q4k_bytes(n, k) for _, n, k in LAYER)

    # Headline: the layer's five Gemv ops as one grouped launch pair per step.
    for i in range(a.warmup):
        run_step_batched(batches[i % COPIES], stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        run_step_batched(batches[i % COPIES], stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    value = weight_bytes * a.steps / dt / 1e9

    # The same five ops launched one by one (one launch each, quantization fused).
    for i in range(a.warmup):
        run_step(S, copies[i % COPIES], xs, ys, wss, stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for i in range(a.steps):
        run_step(S, copies[i % COPIES], xs, ys, wss, stream)
    torch.cuda.synchronize()
    dt_ops = time.perf_counter() - t1

    # Per-launch durations from HIP events on the launching stream: the grouped GEMV launch
    # (the dominant kernel) and, for the one-by-one path, each Gemv op.
    nrep = max(20, min(a.steps, 100))
    for b in batches:
        b.quantize(stream)  # each copy's rows in Q8_K once, outside the timed launches
    for i in range(5):
        batches[i % COPIES].gemv_quantized(stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # a spin kernel first, so every launch below is queued before the GPU reaches it and the
    # event pair times the kernels back to back (launch gaps included), not the host's rate
    torch.cuda._sleep(int(4e7))
    e0.record()
    for i in range(nrep):
        batches[i % COPIES].gemv_quantized(stream)  # k_gemv_q4k_batch alone, back to back
    e1.record()
    torch.cuda.synchronize()
    batch_ms = e0.elapsed_time(e1) / nrep
    ev = [{name: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for name, _, _ in LAYER} for _ in range(nrep)]
    for i in range(nrep):
        run_step(S, copies[i % COPIES], xs, ys, wss, stream, events=ev[i])
    torch.cuda.synchronize()
    per = {name: sum(ev[i][name][0].elapsed_time(ev[i][name][1]) for i in range(nrep)) / nrep
           for name, _, _ in LAYER}  # ms
    # algorithmic bytes of one k_gemv_q4k_batch launch: the weights, each Q8_K row once (codes,
    # 32-value sums, scales) and the F32 outputs
    alg_bytes = sum(q4k_bytes(n, k) + k + k // 8 + k // 64 + 4 * n for _, n, k in LAYER)
    achieved = alg_bytes / (batch_ms * 1e-3) / 1e9

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_q4k_gemv_decode_layer.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt / a.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32, f32 terms",
        "data": "synthetic: W ~ N(0,0.02) -> Q4_K (GPU packer, ggml-exact); x ~ N(0,1) F32",
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
            "one_op_per_launch_us": {k: round(v * 1e3, 3) for k, v in per.items()},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_gemv_q4k_batch<X8> (syn_gemv_batch_quantized_layout: the grouped GEMV on Q8_K rows)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "alg_bytes_per_launch": alg_bytes,
            "avg_launch_us": round(batch_ms * 1e3, 3),
        },
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(torch, copies, xs, a.cpu_seconds)
    del copies, batches
    if not a.no_moe:
        torch.cuda.empty_cache()
        out["moe"] = bench_moe(torch, S, M, max(10, a.steps // 4), max(3, a.warmup // 4),
                               0 if a.no_cpu else a.cpu_seconds)
    if not a.no_prefill:
        torch.cuda.empty_cache()
        out["prefill"] = bench_prefill(torch, S, M, max(5, a.steps // 20), max(2, a.warmup // 10),
                                       0 if a.no_cpu else min(a.cpu_seconds, 5.0))
    print(json.dumps(out))


if __name__ == "__main__":
    main()
