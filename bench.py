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
  roofline      the dominant kernel (gate/up) on its binding roofline (HBM),
                from HIP-event timing of back-to-back launches on the launch stream
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


def time_operations(layers, steps: int, torch) -> dict[str, float]:
    """Average duration (ms) of every operation of a layer call, from HIP events
    recorded between the operations of whole eager layer calls on the stream
    they are launched on (torch's current stream). Operations always run in
    order: their inputs are the previous operations' outputs, and the packed
    workspace lets a later operation's tensors reuse an earlier one's bytes,
    so an operation launched on its own would read stale data."""
    names = layers[0].op_names
    for lay in layers:
        lay.forward()
    torch.cuda.synchronize()
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(steps)]
    for i in range(steps):
        lay = layers[i % len(layers)]
        marks[i][0].record()
        for j, op in enumerate(names):
            lay.run_operation(op)
            marks[i][j + 1].record()
    torch.cuda.synchronize()
    return {op: sum(m[j].elapsed_time(m[j + 1]) for m in marks) / steps for j, op in enumerate(names)}


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
            kern["isolated"] = {op: time_isolated(xl, op, max(50, steps // 2), torch) * 1e3 for op in ISOLATED_OPS}
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
    dom_op, dom_us = "gate_up", iso["gate_up"]
    dom_bytes = gate_up_bytes(cfg, touched, path)
    dn_us, dn_bytes = iso["down"], down_bytes(cfg, touched, path)
    other = {"down": {"achieved_gbps": dn_bytes / (dn_us * 1e-6) / 1e9, "avg_us": dn_us,
                      "algorithmic_bytes_per_launch": dn_bytes}}
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
        "cpu_baseline": cpu, "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
