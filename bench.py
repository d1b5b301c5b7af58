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
launches / their time.  roofline.traffic: measured HBM bytes per dominant
launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy) read
from the committed summary that `--traffic-run` / `--traffic-summary` make.
cpu_baseline: the NumPy oracle (a restatement of the reference
decomposition) on a bounded sample, on this host's cores.
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
PEAK = {"bf16": 2500.0, "fp16": 2500.0, "fp8": 5000.0, "int8": 5000.0, "fp32": 157.3, "hbm": 8000.0}
# Dominant kernel family and its roofline per workload.
DOMINANT = {
    "mlp": (["gemm", "splitk_reduce"], "fp32", "fp32 GEMM, split-K partials + ordered reduce (MFMA 16x16x4 f32)"),
    "resnet18_cifar": (["conv"], "fp32", "implicit-GEMM conv (fp32 MFMA)"),
    "resnet18_224": (["conv"], "bf16", "implicit-GEMM conv (bf16 MFMA 16x16x32)"),
    "decoder_fp16": (["gemm"], "fp16", "GEMM + fused epilogues (fp16 MFMA 16x16x32)"),
    "decoder_w8a8": (["qgemm"], "int8", "int8 GEMM + requant/dequant epilogue (MFMA i32 16x16x64)"),
    "decoder_fp8": (["gemm_fp8"], "fp8", "E4M3 GEMM + scale/epilogue (MFMA f32 16x16x128 f8f6f4)"),
}
BASELINE_INDEX = {"mlp": 0, "resnet18_cifar": 1, "resnet18_224": 2, "decoder_fp16": 3, "decoder_w8a8": 4}
CPU_SAMPLE = {"mlp": 4096, "resnet18_cifar": 128, "resnet18_224": 48, "decoder_fp16": 16, "decoder_w8a8": 2}
# decoder_fp8 is no BASELINE config: the decoder_fp16 model under the "fp8" policy (E4M3 GEMMs).


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _prepare(name: str):
    from hackathon_amd.workloads import compile_workload

    return compile_workload(name)


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


# -- HBM traffic of the dominant kernel (two rocprofv3 --pmc passes) -------------------------------
COPY_BYTES = 1 << 30
TRAFFIC_PROFILE = ROOT / "profiles" / f"{HEADLINE}_conv_traffic.md"


def _traffic_run(meta_path: str, reps: int = 3) -> int:
    """The dispatch stream the FETCH_SIZE and WRITE_SIZE passes count.

    First a plain copy of COPY_BYTES (strided_copy_kernel, 8-byte elements,
    dense): what the counters read for it against the bytes it must move is
    the calibration factor.  Then the headline workload's dominant launches
    (every conv of one step) replayed `reps` + 1 times as a hipGraph; the
    per-launch algorithmic bytes go to `meta_path` for the summary."""
    import numpy as np

    from hackathon_amd.c35 import engine
    from hackathon_amd.device import DeviceArray, init, synchronize

    init(0)
    n = COPY_BYTES // 8
    src, dst = DeviceArray.empty((n,), np.int64), DeviceArray.empty((n,), np.int64)
    for _ in range(3):
        engine.strided_copy(src, dst, (n,), (1,))
    synchronize()
    del src, dst
    m, plan, prog = _prepare(HEADLINE)
    idx = prog.launches_of(DOMINANT[HEADLINE][0])
    prog.time_subset(idx, reps=reps)
    synchronize()
    meta = {"workload": HEADLINE, "copy_bytes": COPY_BYTES, "copy_dispatches": 3, "replays": reps + 1,
            "launches": [{k: prog.launch_meta[i][k] for k in ("kind", "flops", "bytes")} for i in idx]}
    with open(meta_path, "w") as f:
        json.dump(meta, f, indent=1)
    _log(f"traffic run: {len(idx)} dominant launches x {reps + 1} replays, meta -> {meta_path}")
    return 0


def _pmc_rows(run_dir: str, counter: str):
    """(kernel name, value in KiB) per dispatch, in dispatch order, from a rocprofv3 csv directory."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *counter_collection.csv under {run_dir}")
    rows = []
    for path in files:
        with open(path) as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def _traffic_summary(fetch_dir: str, write_dir: str, meta_path: str) -> int:
    """Calibrated HBM bytes per dominant launch -> profiles/<headline>_conv_traffic.md."""
    import numpy as np

    with open(meta_path) as f:
        meta = json.load(f)
    launches = meta["launches"]
    out = {}
    for counter, run_dir in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _pmc_rows(run_dir, counter)
        copy = [v for k, v in rows if "strided_copy_kernel" in k]
        conv = [v for k, v in rows if "mfma_gemm" in k or "conv_stem_pool" in k or "conv3x3_c64" in k]
        if len(copy) != meta["copy_dispatches"] or len(conv) != len(launches) * meta["replays"]:
            raise ValueError(f"{counter}: {len(copy)} copy / {len(conv)} conv dispatches, expected "
                             f"{meta['copy_dispatches']} / {len(launches) * meta['replays']}")
        factor = meta["copy_bytes"] / (float(np.median(copy)) * 1024.0)
        per = np.asarray(conv).reshape(meta["replays"], len(launches)).mean(axis=0) * 1024.0 * factor
        out[counter] = (factor, float(np.median(copy)), per)
    f_fac, f_copy, fetch = out["FETCH_SIZE"]
    w_fac, w_copy, write = out["WRITE_SIZE"]
    alg = np.asarray([l["bytes"] for l in launches], float)
    traffic = fetch + write
    lines = [
        f"# {meta['workload']}: HBM traffic of the implicit-GEMM conv launches (rocprofv3 --pmc)", "",
        "Commands (repository root, MI355X box; one counter per pass):", "", "```",
        "timeout -s KILL 180 rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch -o run -- \\",
        "    python3 bench.py --traffic-run gpurun_out/traffic_meta_fetch.json",
        "timeout -s KILL 180 rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write -o run -- \\",
        "    python3 bench.py --traffic-run gpurun_out/traffic_meta.json",
        "python3 bench.py --traffic-summary gpurun_out/pmc_fetch gpurun_out/pmc_write gpurun_out/traffic_meta.json",
        "```", "",
        f"Calibration: a dense copy of {meta['copy_bytes'] / 2**20:.0f} MiB (strided_copy_kernel) reads "
        f"FETCH_SIZE {f_copy:.0f} KiB and WRITE_SIZE {w_copy:.0f} KiB per dispatch; scale factors "
        f"{f_fac:.4f} (fetch) and {w_fac:.4f} (write) turn counter KiB into bytes moved.", "",
        "| launch | algorithmic MB | fetched MB | written MB | traffic / algorithmic |",
        "|---:|---:|---:|---:|---:|",
    ]
    for i in range(len(launches)):
        lines.append(f"| {i} | {alg[i] / 1e6:.1f} | {fetch[i] / 1e6:.1f} | {write[i] / 1e6:.1f} | "
                     f"{traffic[i] / alg[i]:.2f} |")
    lines += ["", f"Per step: algorithmic {alg.sum() / 1e9:.3f} GB, measured {traffic.sum() / 1e9:.3f} GB "
              f"({traffic.sum() / alg.sum():.2f}x).", "",
              f"traffic_bytes_per_launch = {traffic.mean():.0f}",
              f"algorithmic_bytes_per_launch = {alg.mean():.0f}", ""]
    TRAFFIC_PROFILE.write_text("\n".join(lines))
    _log(f"wrote {TRAFFIC_PROFILE}: {traffic.mean() / 1e6:.1f} MB per launch "
         f"({traffic.sum() / alg.sum():.2f}x algorithmic)")
    return 0


def _committed_traffic():
    """HBM bytes per dominant launch from the committed pmc summary, or None."""
    import re

    try:
        m = re.search(r"^traffic_bytes_per_launch = (\d+)$", TRAFFIC_PROFILE.read_text(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="mlp,resnet18_cifar,resnet18_224,decoder_fp16,decoder_w8a8",
                    help="comma-separated workloads to measure (the headline is always included)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-run", metavar="META_JSON",
                    help="dispatch stream for a rocprofv3 --pmc pass (copy calibration + dominant launches)")
    ap.add_argument("--traffic-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "META_JSON"),
                    help="turn the two pmc passes into the committed traffic summary (no GPU)")
    args = ap.parse_args()
    if args.traffic_summary:
        return _traffic_summary(*args.traffic_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.traffic_run:
        return _traffic_run(args.traffic_run)
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
    head["roofline"]["traffic"] = _committed_traffic()
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
