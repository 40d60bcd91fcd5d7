#!/usr/bin/env python3
"""Benchmark of the FP8 routed-MoE layer on one MI355X.

One step = one full layer call (router -> top-k/quant -> sort -> gate/up ->
down -> combine) on inputs already resident in HBM, its kernels dispatched
directly on the stream (--launch eager, the default) or replayed from the
engine's HIP graph (--launch graph). On ROCm 7.2 the direct dispatches
measured faster, host- and GPU-side, than a graph of the same launches: with
the queue kept full, 22.2 against 27.5 us per call at T = 1 and 135.8 against
140.3 us at T = 64. The headline workload is BASELINE config 1 (decode, T=64,
H=2048, 256 routed experts + 1 shared, top-8, I=512). Two copies of the expert
weights alternate between steps so weights stream from HBM rather than the
256 MB last-level cache (T=1, whose call touches only 9 experts, rotates 12
address-distinct copies). The same weights serve the T=1, T=512 (Zipf-skewed)
and T=4096 configs, reported under "secondary", each with its two GEMMs timed
back to back on both rooflines (T=4096: a `roofline` object for gate/up against
dense FP8).

Prints ONE JSON line. Extra objects:
  roofline      the dominant kernel (gate/up; at T=64 the gate/up kernel that
                runs each tile's down too) on its binding roofline (HBM), from
                HIP-event timing of back-to-back launches on the launch stream
  cpu_baseline  the C oracle on the host cores over a bounded token sample
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "netra-kernel_amd"))

HBM_PEAK_GBPS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
WEIGHT_SEED = 77


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gate_up_bytes(cfg, touched: int, path: str) -> int:
    """Algorithmic HBM bytes of one gate/up launch: touched experts' W13 + scales,
    x_q + x scales, and h (e4m3 + 1x128 scales, both paths) for every route row."""
    w = touched * (2 * cfg.I * cfg.H + 4 * (2 * cfg.I // 128) * (cfg.H // 128))
    acts = cfg.T * cfg.H + 4 * cfg.T * (cfg.H // 128)
    outs = cfg.routes * cfg.I + 4 * cfg.routes * (cfg.I // 128)
    return w + acts + outs


def down_bytes(cfg, touched: int, path: str) -> int:
    """Touched experts' W2 + scales, h in, and what the kernel writes: the
    combined bf16 output where the down kernel combines (fused narrow and
    single-token variants), else its route partial rows (fp32 on the fused
    wide and stream paths, bf16 on the tile path), which a combine kernel
    reads back."""
    from netra_moe.engine import down_variant
    w = touched * (cfg.H * cfg.I + 4 * (cfg.H // 128) * (cfg.I // 128))
    h = cfg.routes * cfg.I + 4 * cfg.routes * (cfg.I // 128)
    if path == "fused" and down_variant(cfg) in ("narrow", "single"):
        return w + h + 2 * cfg.T * cfg.H
    part = (2 if path == "tile" else 4) * cfg.routes * cfg.H  # bf16 / fp32 route partials
    return w + h + part


def merged_bytes(cfg, touched: int, path: str) -> int:
    """Algorithmic HBM bytes of one launch of the gate/up kernel that also runs
    each tile's down (the fused path's merged variant): both GEMMs' bytes less
    the h read-back, which stays in the workgroup's LDS."""
    h = cfg.routes * cfg.I + 4 * cfg.routes * (cfg.I // 128)
    return gate_up_bytes(cfg, touched, path) + down_bytes(cfg, touched, path) - h


def gate_up_flops(cfg) -> int:
    """Algorithmic FLOPs of one gate/up launch: 2 * 2I * H per route row."""
    return 2 * cfg.routes * 2 * cfg.I * cfg.H


def down_flops(cfg) -> int:
    return 2 * cfg.routes * cfg.H * cfg.I


# Weight copies a config rotates through, so that its weights come from HBM
# and not from the 256 MB last-level cache: one T = 1 call touches 9 experts
# (28.3 MB), so 12 copies (340 MB between reuses of a copy); the larger
# configs touch 240 MB or more per call and alternate the 2 base copies.
COLD_COPIES = {"decode_t1": 12}


def time_layer(layers, steps: int, warmup: int, torch):
    for i in range(warmup):
        layers[i % len(layers)].forward()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        layers[i % len(layers)].forward()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall * 1e3 / steps


# GPU sleep queued ahead of timed launches, in GPU clock cycles per eight
# launches: longer than the host takes to launch them.
QUEUE_AHEAD_CYCLES = 2_500_000


def time_operations(layers, steps: int, torch) -> dict[str, float]:
    """Marginal GPU time (ms) of every operation of a layer call: the average
    time of `steps` back-to-back eager calls truncated after operation k,
    minus the same for the calls truncated before it, so the figures add up
    to the eager call's time. A truncated call is a valid layer prefix (an
    operation reads only the layer's inputs and the outputs of earlier
    operations of the same call). The launches are queued behind a GPU sleep,
    so the host's launch rate, which exceeds the duration of the short
    routing kernels, is not timed; and no event is recorded between two
    operations (an event between kernels costs GPU time of its own, largest
    after kernels that leave much written data in the L2 caches)."""
    names = layers[0].op_names
    for lay in layers:
        lay.forward()
    torch.cuda.synchronize()
    prefix = [0.0]
    for k in range(1, len(names) + 1):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(QUEUE_AHEAD_CYCLES * max(1, steps * k // 8))
        start.record()
        for i in range(steps):
            lay = layers[i % len(layers)]
            for op in names[:k]:
                lay.run_operation(op)
        end.record()
        torch.cuda.synchronize()
        prefix.append(start.elapsed_time(end) / steps)
    return {op: prefix[j + 1] - prefix[j] for j, op in enumerate(names)}


# Operations that are pure functions of other operations' outputs (nothing
# rewritten in place), so they can be relaunched back to back on a layer whose
# intermediates are all bindings of their own.
ISOLATED_OPS = ("gate_up", "down")


def time_isolated(layers, op: str, steps: int, torch) -> float:
    """Average duration (ms) of back-to-back launches of one GEMM operation
    (HIP events on its stream, torch's current stream) after a whole layer
    call produced its inputs; the layers expose every intermediate, so no
    other operation's tensors share its inputs' bytes."""
    if op not in ISOLATED_OPS:
        raise ValueError(f"{op} is not timed in isolation")
    for lay in layers:
        lay.forward()
    torch.cuda.synchronize()
    for i in range(4):
        layers[i % len(layers)].run_operation(op)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(QUEUE_AHEAD_CYCLES * max(1, steps // 8))  # queue the launches ahead of the GPU
    start.record()
    for i in range(steps):
        layers[i % len(layers)].run_operation(op)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_baseline(cfg, act_cpu, w_host, threads: int, min_seconds: float):
    import numpy as np

    sys.path.insert(0, str(REPO / "oracle"))
    import oracle

    oracle.build()
    x = act_cpu["x"].contiguous().view(__import__("torch").int16).numpy().view(np.uint16)
    rw = act_cpu["router_w"].contiguous().view(__import__("torch").int16).numpy().view(np.uint16)
    bias = act_cpu["router_bias"].numpy()
    n = min(cfg.T, 64)
    xs = np.ascontiguousarray(x[:n])
    runs = []
    t_total = 0.0
    while t_total < min_seconds or len(runs) < 3:
        t0 = time.perf_counter()
        logits = oracle.router_logits(xs, rw, threads)
        ids, wts = oracle.topk(logits, bias, cfg.E, cfg.K, cfg.S)
        x_q, x_s = oracle.quant_rows_bf16(xs)
        oracle.moe_tokens(x_q, x_s, w_host["w13"], w_host["w13_scale"], w_host["w2"], w_host["w2_scale"],
                          ids, wts, np.arange(n, dtype=np.int64), cfg.H, cfg.I, threads)
        dt = time.perf_counter() - t0
        runs.append(dt)
        t_total += dt
        if len(runs) >= 1000:
            break
    med = sorted(runs)[len(runs) // 2]
    host = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host
    return {"value": n / med, "unit": "tokens/s", "cores": threads, "host_cores": host,
            "host_cores_usable": usable, "kind": "port",
            "sample": f"{n} tokens of {cfg.name} (router+top-k+quant+all {cfg.Ktot} expert slots per token, "
                      f"fp64-accumulated C oracle, OpenMP), median of {len(runs)} runs, {med * 1e3:.1f} ms each"}


# The reference's published isolated HIP-event medians for its per-operation
# bridges on MI350X (docs/notes/gfx950-qwen36-fp8-kernels.md lines 78, 261,
# 301, 563, 643), at the shapes they were quoted for. (Its SiLU-quant and
# shared-gate notes also give kernel-trace figures: 2.742 us, line 80, and a
# serving-trace median of 3.160 us, line 263.) The M768 prefill pair has no
# published per-launch time (its notes give serving throughput only).
REFERENCE_BRIDGE_US = {"router_m1": 6.24, "router_m16": 6.32, "shared_gate_m1": 5.96,
                       "silu_mul_quant_m1": 2.78, "gate_up_m1": 8.96, "down_reduce_m1": 10.28}


def bridge_timings(torch, dev, launches: int = 200, copies: int = 12) -> dict:
    """Per-launch HIP-event medians of libnetra_bridges.so at the reference's
    shapes (hidden 2048, 256 routed + 1 shared expert, top-8 + 1, intermediate
    512; weights in the AITER 16x16 shuffle the reference's kernels read).
    "hot" repeats one argument set, the reference's method; "cold" rotates
    `copies` address-distinct copies of the weights the launch streams, so they
    come from HBM and not the last-level cache."""
    import ctypes

    from netra_moe import bridges as B

    H, E, I, K = 2048, 256, 512, 9
    g = torch.Generator(device=dev).manual_seed(5)

    def fp8(*shape):
        return (torch.randn(shape, generator=g, device=dev) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)

    def f32(*shape, scale=1e-3):
        return torch.rand(shape, generator=g, device=dev) * scale + scale

    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    w13, w13s = fp8(E + 1, 2 * I, H), f32(E + 1, 2 * I // 128, H // 128)
    w2, w2s = fp8(E + 1, H, I), f32(E + 1, H // 128, I // 128)
    router = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    shared_w = (torch.randn((1, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((16, H), generator=g, device=dev).to(torch.bfloat16)
    xq, xs = fp8(16, H), f32(16, H // 128, scale=1e-2)
    ids = torch.stack([torch.randperm(E, generator=g, device=dev)[:K - 1] for _ in range(16)]).to(torch.int32)
    ids9 = torch.cat([ids, torch.full((16, 1), E, dtype=torch.int32, device=dev)], 1).contiguous()
    wts9 = torch.softmax(torch.rand((16, K), generator=g, device=dev), 1).contiguous()
    wts8 = wts9[:, :K - 1].contiguous()
    logits = torch.empty((16, E), dtype=torch.bfloat16, device=dev)
    out_ids = torch.empty((16, K), dtype=torch.int32, device=dev)
    out_w = torch.empty((16, K), dtype=torch.float32, device=dev)
    gu = torch.randn((K * 16, 2 * I), generator=g, device=dev)
    hq, hs = torch.empty((K * 16, I), dtype=torch.uint8, device=dev), torch.empty((K * 16, I // 128), device=dev)
    hq.copy_(fp8(K * 16, I))
    out = torch.empty((16, H), dtype=torch.bfloat16, device=dev)
    hot_w = [(w13, w13s, w2, w2s)]
    cold_w = hot_w + [(w13.clone(), w13s.clone(), w2.clone(), w2s.clone()) for _ in range(copies - 1)]
    torch.cuda.synchronize()

    def batch_us(fn, sets):
        """Per-launch GPU time of `launches` back-to-back launches, queued behind
        a GPU sleep so the host's launch latency is not timed (an event pair
        around every launch costs ~6 us on its own at this size)."""
        for i in range(10):
            fn(sets[i % len(sets)])
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(50_000_000)
        a.record()
        for i in range(launches):
            fn(sets[i % len(sets)])
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / launches

    cases = {
        "router_m1": ("netra_qwen36_router_bf16", lambda w: B.launch("netra_qwen36_router_bf16", P(logits), P(x),
                                                                     P(router), 1, stream), False),
        "router_m16": ("netra_qwen36_router_bf16", lambda w: B.launch("netra_qwen36_router_bf16", P(logits), P(x),
                                                                      P(router), 16, stream), False),
        "shared_gate_m1": ("netra_qwen36_shared_gate_append",
                           lambda w: B.launch("netra_qwen36_shared_gate_append", P(out_ids), P(out_w), P(x),
                                              P(shared_w), P(ids), P(wts8), 1, stream), False),
        "silu_mul_quant_m1": ("netra_qwen36_moe_silu_mul_quant",
                              lambda w: B.launch("netra_qwen36_moe_silu_mul_quant", P(gu), P(hq), P(hs), K, stream),
                              False),
        "gate_up_m1": ("netra_qwen36_moe_gate_up",
                       lambda w: B.launch("netra_qwen36_moe_gate_up", P(xq), P(xs), P(w[0]), P(w[1]), P(ids9), P(gu),
                                          1, stream), True),
        "down_reduce_m1": ("netra_qwen36_moe_down_reduce",
                           lambda w: B.launch("netra_qwen36_moe_down_reduce", P(hq), P(hs), P(w[2]), P(w[3]),
                                              P(wts9), P(ids9), P(out), 1, stream), True),
    }
    # The M768 pair (producer + reducer) at its one shape: 768 tokens, their
    # routing and AITER sorted format produced by this build's own screen front
    # end (a T = 768 layer call with its routing tensors exposed).
    from netra_moe.config import MoEConfig
    from netra_moe.layer import MoELayer
    m768 = MoEConfig("m768", T=768, H=H, E=E, K=K - 1, I=I, S=1, seed=1105)
    rw = (torch.randn((E + 1, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    lay = MoELayer(m768, {"router_w": rw, "router_bias": torch.zeros(E, device=dev),
                          "w13": fp8(E + 1, 2 * I, H), "w13_scale": w13s, "w2": fp8(E + 1, H, I), "w2_scale": w2s},
                   graph=False, expose=("sorted_ids", "sorted_expert", "num_valid", "topk_weights", "x_q", "x_scale"))
    lay.x.copy_(torch.randn((768, H), generator=g, device=dev).to(torch.bfloat16))
    lay.forward()
    torch.cuda.synchronize()
    mb = {n: lay.buffer(n).clone() for n in ("sorted_ids", "sorted_expert", "num_valid", "topk_weights", "x_q",
                                             "x_scale")}
    lay.close()
    half = 768 * K + m768.cap_blocks
    m_sw = torch.zeros(m768.cap_rows, device=dev)  # sorted weights: unused by the producer, as in the reference
    m_rs = torch.empty((m768.cap_rows, I // 128), device=dev)
    m_parts = torch.empty((2, half, H), dtype=torch.float16, device=dev)
    m_out = torch.empty((768, H), dtype=torch.bfloat16, device=dev)
    cases["prefill_m768"] = (
        "netra_moe_prefill_m768",
        lambda w: B.launch("netra_moe_prefill_m768", P(mb["x_q"]), P(mb["x_scale"]), P(w[0]), P(w[1]), P(w[2]),
                           P(w[3]), P(mb["sorted_ids"]), P(m_sw), P(mb["sorted_expert"]), P(mb["num_valid"]),
                           P(mb["topk_weights"]), P(m_rs), P(m_parts), P(m_out), stream), True)
    res = {}
    for name, (fam, fn, streams_weights) in cases.items():
        B.check(fam, B.load(fam))
        r = {"hot_us": batch_us(fn, hot_w), "reference_mi350x_us": REFERENCE_BRIDGE_US.get(name)}
        if streams_weights:
            r["cold_us"] = batch_us(fn, cold_w)
        B.check(fam, B.unload(fam))
        res[name] = r
    res["method"] = (f"HIP events around {launches} back-to-back launches (after 10 warm-up launches), queued "
                     f"behind a GPU sleep so no host gap is timed, per launch (kernel plus the gap to the next); "
                     f"hot: one argument set (the reference's method); cold: {copies} address-distinct weight "
                     f"copies rotated. Kernel-only durations: profiles/bridges_kernel_stats.md")
    del cold_w
    torch.cuda.empty_cache()
    return res


COPY_BYTES = 1 << 30
PMC_REPS = 6


def copy_probe(W, torch, dev, reps: int = 10) -> float:
    """GB/s of the library's plain copy kernel over 1 GiB (read + write bytes)."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    W.device_copy(src, dst)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        W.device_copy(src, dst)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    del src, dst
    return 2 * COPY_BYTES / (ms / 1e3) / 1e9


def pmc_workload(cfg_name: str) -> int:
    """Run under rocprofv3 --pmc: three calibration copies of COPY_BYTES, then
    PMC_REPS direct (non-graph) layer calls, each operation a dispatch of its own."""
    import torch

    from netra_moe import weights as W
    from netra_moe.config import BASELINE_CONFIGS
    from netra_moe.layer import MoELayer

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = BASELINE_CONFIGS[cfg_name]
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        W.device_copy(src, dst)
    torch.cuda.synchronize()
    del src, dst
    ws = W.synthetic_expert_weights(cfg, WEIGHT_SEED, dev)
    act = W.synthetic_activations(cfg, dev)
    lay = MoELayer(cfg, {"router_w": act["router_w"], "router_bias": act["router_bias"], **ws}, graph=False)
    lay.x.copy_(act["x"])
    for _ in range(PMC_REPS):
        lay.forward()
    torch.cuda.synchronize()
    lay.close()
    log(f"[pmc-workload] {cfg_name}: done")
    return 0


def read_counter_csv(directory: Path, counter: str) -> dict[str, list[float]]:
    """{kernel name: [per-dispatch value]} from a rocprofv3 counter_collection csv."""
    import csv

    files = sorted(directory.rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {directory}")
    out: dict[str, list[float]] = {}
    for f in files:
        with f.open() as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                out.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return out


def measure_traffic(cfg_name: str, kernel_prefix: str, out_dir: Path) -> dict:
    """HBM bytes per launch of the first kernel whose name starts with
    kernel_prefix, from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, KiB
    per dispatch) over a child process running pmc_workload, each scaled by the
    same counter's reading for the calibration copy of COPY_BYTES bytes."""
    import shutil
    import subprocess

    exe = shutil.which("rocprofv3")
    if exe is None:
        raise FileNotFoundError("rocprofv3 not on PATH")
    res = {"kernel": None, "counters": {}}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = out_dir / f"pmc_{counter.lower()}"
        shutil.rmtree(d, ignore_errors=True)
        cmd = ["timeout", "-s", "KILL", "240", exe, "--pmc", counter, "--output-format", "csv",
               "-d", str(d), "-o", "pmc", "--", sys.executable, "-u", str(Path(__file__).resolve()),
               "--pmc-workload", "--config", cfg_name]
        log(f"[bench] counter pass {counter}: {' '.join(cmd)}")
        proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        vals = read_counter_csv(d, counter)  # results are whole even if the profiler exits non-zero
        copy = [v for k, v in vals.items() if k.startswith("netra_moe_copy_gfx950")]
        kern = [(k, v) for k, v in vals.items() if k.startswith(kernel_prefix)]
        if not copy or not kern:
            raise RuntimeError(f"{counter}: kernels missing from the counter csv (rc {proc.returncode})")
        copy_kib = sorted(copy[0])[len(copy[0]) // 2]
        name, kv = kern[0]
        kib = sorted(kv)[len(kv) // 2]
        factor = COPY_BYTES / copy_kib  # bytes per counter unit, from the copy
        res["kernel"] = name
        res["counters"][counter] = {"kernel_kib_median": kib, "dispatches": len(kv),
                                    "copy_kib_median": copy_kib, "bytes_per_unit": factor,
                                    "bytes": kib * factor}
    res["bytes"] = res["counters"]["FETCH_SIZE"]["bytes"] + res["counters"]["WRITE_SIZE"]["bytes"]
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode_t64")
    ap.add_argument("--secondary", default="decode_t1,verify_t512,prefill_t4096",
                    help="comma-separated extra configs with the same dims ('' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure the dominant kernel's HBM bytes")
    ap.add_argument("--no-bridges", action="store_true", help="skip timing the per-operation bridges")
    ap.add_argument("--bridges-only", action="store_true",
                    help="time only the per-operation bridges (one JSON line), e.g. under a kernel trace")
    ap.add_argument("--launch", choices=("eager", "graph"), default="eager",
                    help="dispatch each layer call's kernels directly, or replay the engine's HIP graph")
    ap.add_argument("--pmc-workload", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design "
                          "note (expert parallel over RCCL), not implemented", "n_gpus": args.gpus}))
        return 2
    if args.pmc_workload:
        return pmc_workload(args.config)
    if args.bridges_only:
        import torch
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        print(json.dumps({"bridges": bridge_timings(torch, dev)}), flush=True)
        return 0

    import numpy as np
    import torch

    from netra_moe import weights as W
    from netra_moe.config import BASELINE_CONFIGS
    from netra_moe.engine import operations, resolve_path
    from netra_moe.layer import MoELayer

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = BASELINE_CONFIGS[args.config]
    path = resolve_path(cfg)
    copy_gbps = copy_probe(W, torch, dev)
    log(f"[bench] copy kernel: {copy_gbps:.0f} GB/s (read + write)")
    log(f"[bench] weights: 2 copies of {cfg.Etot} experts ({2 * cfg.Etot * cfg.expert_bytes() / 1e9:.2f} GB)")
    # copy 0 also keeps its row-major bytes: the CPU baseline reads that layout
    wsets = [W.synthetic_expert_weights(cfg, WEIGHT_SEED + i, dev, keep_row_major=(i == 0))
             for i in range(2)]
    torch.cuda.synchronize()

    def copies_for(c):
        """The weight sets a config rotates through: the 2 base copies, or for
        configs that touch few experts per call, byte-identical clones of them
        at other addresses (caches key on addresses; routing does not depend
        on the expert weights)."""
        n = COLD_COPIES.get(c.name, len(wsets))
        out = []
        for i in range(n):
            base = wsets[i % len(wsets)]
            out.append(base if i < len(wsets) else
                       {k: v.clone() for k, v in base.items() if k in ("w13", "w13_scale", "w2", "w2_scale")})
        return out

    def run_config(c, steps, warmup, with_kernels):
        act = W.synthetic_activations(c, "cpu")
        sets = copies_for(c)
        layers = []
        for ws in sets:
            w = {"router_w": act["router_w"].to(dev).clone(), "router_bias": act["router_bias"].to(dev), **ws}
            lay = MoELayer(c, w, expose=("topk_ids",), graph=args.launch == "graph")
            lay.x.copy_(act["x"].to(dev))
            layers.append(lay)
        ms, wall_ms = time_layer(layers, steps, warmup, torch)
        ids = layers[0].buffer("topk_ids").cpu().numpy()
        touched = int(np.unique(ids).size)
        flops = c.flops()
        nbytes = c.algorithmic_bytes(touched)
        res = {"T": c.T, "gemm_path": resolve_path(c), "ms_per_step": ms, "wall_ms_per_step": wall_ms,
               "tokens_per_s": c.T / (ms / 1e3), "tflops": flops / (ms / 1e3) / 1e12,
               "gbps": nbytes / (ms / 1e3) / 1e9, "touched_experts": touched,
               "algorithmic_bytes": nbytes, "flops": flops, "weight_copies_rotated": len(sets)}
        res["hbm_frac"] = res["gbps"] / HBM_PEAK_GBPS
        res["mfma_frac"] = res["tflops"] / FP8_PEAK_TFLOPS
        kern = None
        if with_kernels:
            dl = []
            for ws in sets:
                w = {"router_w": act["router_w"].to(dev).clone(), "router_bias": act["router_bias"].to(dev), **ws}
                lay = MoELayer(c, w, graph=False)
                lay.x.copy_(act["x"].to(dev))
                dl.append(lay)
            kern = {op: ms * 1e3 for op, ms in time_operations(dl, max(50, steps // 2), torch).items()}  # us
            for lay in dl:
                lay.close()
            # the GEMMs' own durations, for the rooflines
            from netra_moe.engine import tensor_table
            inter = tuple(n for n, sp in tensor_table(c).items() if sp.role == "temporary")
            xl = []
            for ws in sets:
                w = {"router_w": act["router_w"].to(dev).clone(), "router_bias": act["router_bias"].to(dev), **ws}
                lay = MoELayer(c, w, graph=False, expose=inter)
                lay.x.copy_(act["x"].to(dev))
                xl.append(lay)
            kern["isolated"] = {op: time_isolated(xl, op, max(50, steps // 2), torch) * 1e3
                                for op in ISOLATED_OPS if op in xl[0].op_names}
            for lay in xl:
                lay.close()
        for lay in layers:
            lay.close()
        del sets
        torch.cuda.empty_cache()
        return res, kern, act

    log(f"[bench] {cfg.name}: warmup {args.warmup}, steps {args.steps}")
    main_res, kern, act = run_config(cfg, args.steps, args.warmup, True)
    touched = main_res["touched_experts"]
    iso = kern.pop("isolated")
    from netra_moe.engine import down_variant
    merged = path == "fused" and down_variant(cfg) == "merged"  # gate/up runs each tile's down too
    dom_op, dom_us = "gate_up", iso["gate_up"]
    dom_bytes = (merged_bytes if merged else gate_up_bytes)(cfg, touched, path)
    other = {}
    if not merged:
        dn_us, dn_bytes = iso["down"], down_bytes(cfg, touched, path)
        other["down"] = {"achieved_gbps": dn_bytes / (dn_us * 1e-6) / 1e9, "avg_us": dn_us,
                         "algorithmic_bytes_per_launch": dn_bytes}
    gu_symbol = next(op["symbol"] for op in operations(cfg, path) if op["name"] == f"moe.{dom_op}")
    roof = {"kernel": gu_symbol, "bound": "hbm",
            "achieved": dom_bytes / (dom_us * 1e-6) / 1e9, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "traffic": None, "avg_us": dom_us, "algorithmic_bytes_per_launch": dom_bytes,
            "box_copy_gbps": copy_gbps}
    roof["frac"] = roof["achieved"] / roof["peak"]

    def gemm_rooflines(c, touched, iso):
        """The two GEMMs of config c, timed back to back (HIP events on their
        stream), on both rooflines: algorithmic FLOPs against dense FP8 and
        algorithmic bytes against HBM."""
        p = resolve_path(c)
        syms = {op["name"]: op["symbol"] for op in operations(c, p)}
        out = {}
        for op, fl, by in (("gate_up", gate_up_flops(c), gate_up_bytes(c, touched, p)),
                           ("down", down_flops(c), down_bytes(c, touched, p))):
            if op not in iso:  # the merged decode variant: no down launch
                continue
            us = iso[op]
            out[op] = {"kernel": syms[f"moe.{op}"], "avg_us": us, "flops": fl, "bytes": by,
                       "tflops": fl / (us * 1e-6) / 1e12, "gbps": by / (us * 1e-6) / 1e9}
            out[op]["mfma_frac"] = out[op]["tflops"] / FP8_PEAK_TFLOPS
            out[op]["hbm_frac"] = out[op]["gbps"] / HBM_PEAK_GBPS
        return out

    secondary = {}
    for name in [s for s in args.secondary.split(",") if s]:
        c = BASELINE_CONFIGS[name]
        log(f"[bench] secondary {name}")
        # at least 50 timed steps and 10 warm-up steps, whatever --steps says
        res, kern_c, _ = run_config(c, max(50, args.steps), max(10, args.warmup), True)
        iso_c = kern_c.pop("isolated")
        res["kernels_us"] = kern_c
        res["gemms"] = gemm_rooflines(c, res["touched_experts"], iso_c)
        if c.name == "prefill_t4096":  # the north star's MFMA bar: the dominant GEMM on dense FP8
            g = res["gemms"]["gate_up"]
            res["roofline"] = {"kernel": g["kernel"], "bound": "mfma", "achieved": g["tflops"],
                               "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": g["mfma_frac"],
                               "avg_us": g["avg_us"], "algorithmic_flops_per_launch": g["flops"],
                               "hbm": {"achieved": g["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                                       "frac": g["hbm_frac"], "algorithmic_bytes_per_launch": g["bytes"]},
                               "traffic": None}
        secondary[name] = res

    bridges = None
    if not args.no_bridges:
        log("[bench] per-operation bridges")
        bridges = bridge_timings(torch, dev)

    cpu = None
    if not args.no_cpu_baseline:
        # the GPU box grants one GPU's share of its host: 16 threads at most,
        # whatever nproc shows (the line reports both)
        threads = min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1)
        log(f"[bench] cpu baseline on {threads} threads (host nproc {os.cpu_count()})")
        w_host = {"w13": wsets[0]["w13_row_major"].cpu().numpy(),
                  "w13_scale": wsets[0]["w13_scale"].cpu().numpy(),
                  "w2": wsets[0]["w2_row_major"].cpu().numpy(),
                  "w2_scale": wsets[0]["w2_scale"].cpu().numpy()}
        cpu = cpu_baseline(cfg, act, w_host, threads, args.cpu_seconds)

    if not args.no_traffic:
        del wsets
        torch.cuda.empty_cache()
        try:
            t = measure_traffic(cfg.name, gu_symbol, REPO / "gpurun_out" / "bench_pmc")
            roof["traffic"] = t["bytes"]
            roof["traffic_detail"] = t
        except Exception as exc:  # counters unavailable: traffic stays null, the reason is reported
            roof["traffic_error"] = f"{type(exc).__name__}: {exc}"
            log(f"[bench] traffic not measured: {roof['traffic_error']}")

    line = {
        "metric": "MoE layer tokens/s, decode T=64 (H=2048, 256 routed + 1 shared expert, top-8, I=512, "
                  "FP8 E4M3 128x128/1x128 block scales)",
        "value": main_res["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": main_res["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3", "data": "synthetic (seeded)",
        "config": {"workload": cfg.name, "T": cfg.T, "H": cfg.H, "E": cfg.E, "K": cfg.K, "S": cfg.S,
                   "I": cfg.I, "block_m": 64, "weight_copies_rotated": main_res["weight_copies_rotated"],
                   "launch": args.launch},
        "layer": main_res, "kernels_us": kern, "roofline": roof, "other_kernels": other,
        "cpu_baseline": cpu, "secondary": secondary, "bridges": bridges,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
