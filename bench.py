"""Throughput of the compiled HIP execution path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs a,b,...] [--no-cpu-baseline]

A step is one forward pass of a workload over one batch of synthetic,
seeded input already resident in HBM: the whole compiled program (every
launch of the plan) replayed as one hipGraph on the compiled stream.  The
JSON line's headline is ResNet-18 224x224 bf16 at batch 256, the workload
whose conv-GEMM MFMA utilisation is the stated target; every other
configuration is measured the same way under "per_config".

roofline: the dominant kernel family of the workload (conv for ResNet,
16-bit GEMM for the fp16 decoder, int8 GEMM for W8A8, fp32 GEMM for the
MLP) is replayed alone as a hipGraph of just those launches, timed with HIP
events on the compiled stream; achieved = algorithmic flops of those
launches / their time.  cpu_baseline: the NumPy oracle (a restatement of
the reference decomposition) on a bounded sample, on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "samples/s (tokens/s) @1 GPU per config; % of MFMA or HBM roofline per kernel"
HEADLINE = "resnet18_224"
# MI355X published dense peaks (TFLOP/s or TOP/s) and HBM bandwidth (GB/s).
PEAK = {"bf16": 2500.0, "fp16": 2500.0, "int8": 5000.0, "fp32": 157.3, "hbm": 8000.0}
# Dominant kernel family and its roofline per workload.
DOMINANT = {
    "mlp": (["gemm"], "fp32", "fp32 GEMM (MFMA 16x16x4 f32)"),
    "resnet18_cifar": (["conv"], "fp32", "implicit-GEMM conv (fp32 MFMA)"),
    "resnet18_224": (["conv"], "bf16", "implicit-GEMM conv (bf16 MFMA 16x16x32)"),
    "decoder_fp16": (["gemm"], "fp16", "GEMM + fused epilogues (fp16 MFMA 16x16x32)"),
    "decoder_w8a8": (["qgemm"], "int8", "int8 GEMM + requant/dequant epilogue (MFMA i32 16x16x64)"),
}
BASELINE_INDEX = {"mlp": 0, "resnet18_cifar": 1, "resnet18_224": 2, "decoder_fp16": 3, "decoder_w8a8": 4}
CPU_SAMPLE = {"mlp": 256, "resnet18_cifar": 16, "resnet18_224": 8, "decoder_fp16": 8, "decoder_w8a8": 1}


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _prepare(name: str):
    from hackathon_amd import models
    from hackathon_amd.c32.strategy import PrecisionPolicy
    from hackathon_amd.c33.pipeline import GraphPassPipeline
    from hackathon_amd.c34.scheduler import ExecutionScheduler
    from hackathon_amd.c35.compiled import CompiledPlan
    from hackathon_amd.c35.executor import load_weights, fold_conv_batchnorm

    m = models.build(name)
    GraphPassPipeline().run(m.graph)
    host_w, host_c = load_weights(m.weights)
    host_w.update(fold_conv_batchnorm(m.graph, host_w))
    batch = next(iter(m.inputs.values())).shape[0]
    plan = ExecutionScheduler(m.graph, batch_size=batch, precision_policy=PrecisionPolicy(m.precision)).build()
    prog = CompiledPlan(m.graph, plan, host_w, host_c, policy=m.precision)
    return m, plan, prog


def _measure(name: str, steps: int, warmup: int) -> dict:
    import numpy as np

    from hackathon_amd.device import Event, synchronize

    t0 = time.time()
    m, plan, prog = _prepare(name)
    batch = next(iter(m.inputs.values())).shape[0]
    units = batch * (m.tokens_per_sample if m.unit == "tokens" else 1)
    prog.stage_inputs(m.inputs)
    for _ in range(max(warmup, 1)):
        prog.launch()
    prog.stream.synchronize()
    _log(f"{name}: compiled {prog.num_launches} launches, slab {prog.slab_bytes / 2**20:.0f} MiB "
         f"(setup {time.time() - t0:.1f}s)")
    start, end = Event(timing=True), Event(timing=True)
    synchronize()
    w0 = time.perf_counter()
    start.record(prog.stream)
    for _ in range(steps):
        prog.launch()
    end.record(prog.stream)
    synchronize()
    wall = time.perf_counter() - w0
    gpu_ms = start.elapsed_ms(end)
    out = {k: v.get() for k, v in prog.output_arrays.items()}
    finite = all(bool(np.isfinite(v).all()) for v in out.values())
    kinds, dtype, desc = DOMINANT[name]
    idx = prog.launches_of(kinds)
    k_ms = prog.time_subset(idx, reps=max(5, min(steps, 50)))
    flops, nbytes = prog.work(idx)
    achieved = flops / (k_ms * 1e-3) / 1e12 if k_ms > 0 else 0.0
    res = {
        "value": units * steps / wall,
        "unit": f"{m.unit}/s",
        "ms_per_step": wall * 1e3 / steps,
        "gpu_ms_per_step": gpu_ms / steps,
        "batch": batch,
        "policy": m.precision,
        "launches": prog.num_launches,
        "outputs_finite": finite,
        "roofline": {
            "bound": "mfma", "achieved": achieved, "peak": PEAK[dtype], "unit": "TFLOP/s",
            "frac": achieved / PEAK[dtype], "traffic": None, "kernel": desc,
            "launches_per_step": len(idx), "kernel_ms_per_step": k_ms,
            "avg_launch_us": k_ms * 1e3 / max(1, len(idx)), "flops_per_step": flops,
            "algorithmic_bytes_per_step": nbytes,
            "share_of_step": k_ms / (gpu_ms / steps) if gpu_ms > 0 else None,
        },
    }
    _log(f"{name}: {res['value']:.1f} {res['unit']}, {res['ms_per_step']:.3f} ms/step, "
         f"{desc}: {achieved:.1f} TFLOP/s ({100 * achieved / PEAK[dtype]:.1f}% of peak)")
    del prog
    return res


def _cpu_baseline(name: str) -> dict:
    """The NumPy oracle on a bounded sample of the same workload (median of 3 after a warm-up)."""
    import numpy as np

    from hackathon_amd import models
    from hackathon_amd.c32.strategy import PrecisionPolicy
    from hackathon_amd.c33.pipeline import GraphPassPipeline
    from hackathon_amd.c34.scheduler import ExecutionScheduler
    from oracle import graph_ref

    m = models.build(name)
    GraphPassPipeline().run(m.graph)
    w = {**m.weights, **graph_ref.fold_conv_bn(m.graph, m.weights)}
    b = CPU_SAMPLE[name]
    plan = ExecutionScheduler(m.graph, batch_size=b, precision_policy=PrecisionPolicy(m.precision)).build()
    feed = {k: v[:b] for k, v in m.inputs.items()}
    graph_ref.run_plan(plan, m.graph, w, feed, policy=m.precision)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        graph_ref.run_plan(plan, m.graph, w, feed, policy=m.precision)
        times.append(time.perf_counter() - t0)
        if times[-1] > 60:
            break
    t = float(np.median(times))
    units = b * (m.tokens_per_sample if m.unit == "tokens" else 1)
    affinity = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS", affinity))
    return {"value": units / t, "unit": f"{m.unit}/s", "cores": min(threads, affinity), "kind": "port",
            "sample": f"oracle.graph_ref.run_plan (NumPy restatement of the reference decomposition, "
                      f"{m.precision} policy rounding emulated in fp32) on the first {b} samples of the "
                      f"batch, median of {len(times)} runs ({t:.2f} s each)"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="mlp,resnet18_cifar,resnet18_224,decoder_fp16,decoder_w8a8",
                    help="comma-separated workloads to measure (the headline is always included)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    from hackathon_amd.device import device_props, init

    init(0)
    props = device_props(0)
    _log(f"device: {props.name.decode()} {props.arch.decode()} CUs={props.compute_units}")
    names = [n for n in args.configs.split(",") if n]
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    per = {}
    for n in names:
        per[n] = _measure(n, args.steps, args.warmup)
    head = per[HEADLINE]
    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = _cpu_baseline(HEADLINE)
        _log(f"cpu baseline: {cpu['value']:.2f} {cpu['unit']} on {cpu['cores']} threads ({time.time() - t0:.0f}s)")
    line = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) images, "
        "seeded random-init weights of the named architecture)",
        "config": {"workload": "resnet18_224_bf16", "baseline_config_index": BASELINE_INDEX[HEADLINE],
                   "batch": head["batch"], "input": [3, 224, 224], "policy": "bf16", "parallelism": "single GPU"},
        "roofline": head["roofline"], "cpu_baseline": cpu,
        "per_config": {n: {k: v for k, v in r.items()} for n, r in per.items() if n != HEADLINE},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
