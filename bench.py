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
decomposition) on a bounded sample, on this host's cores -- for the headline
and for every per_config entry, with the thread settings and NumPy's BLAS.

memory_bound (per config): every HBM-bound kernel family on that config's
path (LayerNorm, gather + positional add, quantize, argmax, pooling, ...)
replayed alone as a hipGraph, its algorithmic bytes (each operand read once,
each output written once) over its time: achieved GB/s and the fraction of
MI355X's 8 TB/s, beside what a device-to-device copy of the same bytes
reaches in the same replay.  end_to_end (per config): the same program fed
from and drained to pinned host memory every step (H2D, program, D2H
serialized on one stream); end_to_end_overlapped: load_and_infer's streamed
pipeline over three batches (host I/O overlapped with the GPU, logits
written to a memory-mapped .npy).  Both are PCIe-inclusive rates, reported
beside `value`, never as it.
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
    "decoder_fp4": (["gemm_w4a16"], "fp16", "W4A16 GEMM: MXFP4 weights widened to fp16 in registers "
                    "(fp16 MFMA 16x16x32)"),
}
# profiles/<workload>_<label>.md of each workload's dominant family
PROFILE_LABEL = {"mlp": "gemm", "resnet18_cifar": "conv", "resnet18_224": "conv", "decoder_fp16": "gemm",
                 "decoder_w8a8": "qgemm", "decoder_fp8": "gemm", "decoder_fp4": "w4a16"}
BASELINE_INDEX = {"mlp": 0, "resnet18_cifar": 1, "resnet18_224": 2, "decoder_fp16": 3, "decoder_w8a8": 4}
CPU_SAMPLE = {"mlp": 4096, "resnet18_cifar": 128, "resnet18_224": 48, "decoder_fp16": 16, "decoder_w8a8": 2}
# smaller samples for the per-config baselines (a few seconds of CPU each)
CPU_SAMPLE_PER_CONFIG = {"mlp": 4096, "resnet18_cifar": 32, "resnet18_224": 8, "decoder_fp16": 8, "decoder_w8a8": 1}
# (argmax_finish is not timed alone: it reads the block maxima its GEMM writes in the same replay, which a
# standalone replay of the family would find overwritten by later launches' slab data.)
MEMORY_BOUND = ("layernorm", "layernorm_q", "gather_add", "gather", "quantize", "quantize_fp8", "dequantize", "argmax",
                "maxpool", "gap", "layout", "splitk_reduce", "ew", "softmax", "cast", "copy")
# decoder_fp8 and decoder_fp4 are no BASELINE configs: the decoder_fp16 model under the "fp8" policy
# (E4M3 GEMMs) and the "fp4" policy (W4A16 GEMMs, the reference's fp4 choice made executable).


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
    res["memory_bound"] = _memory_bound(prog, reps=max(5, min(steps, 20)))
    res["end_to_end"] = _end_to_end(prog, m, units, steps=max(3, min(steps, 10)))
    del prog
    res["end_to_end_overlapped"] = _end_to_end_overlapped(name)
    _log(f"{name}: {res['value']:.1f} {res['unit']}, {res['ms_per_step']:.3f} ms/step, "
         f"{desc}: {achieved:.1f} TFLOP/s ({100 * achieved / PEAK[dtype]:.1f}% of peak); "
         f"with host transfers {res['end_to_end']['value']:.1f} {res['unit']} serialized, "
         f"{res['end_to_end_overlapped']['value']:.1f} {res['unit']} overlapped")
    for kind, mb in res["memory_bound"].items():
        _log(f"  {name} {kind}: {mb['launches_per_step']} launches, {mb['us_per_launch']:.1f} us, "
             f"{mb['algorithmic_MB_per_launch']:.1f} MB -> {mb['achieved_GBps']:.0f} GB/s "
             f"({100 * mb['frac_of_hbm_peak']:.1f}% of 8 TB/s; a copy of the same bytes "
             f"{mb['copy_same_bytes_GBps']:.0f} GB/s)")
    return res


def _copy_ms(nbytes: int, count: int, reps: int) -> float:
    """Milliseconds per device-to-device copy moving `nbytes` (nbytes / 2 read, nbytes / 2 written), timed as
    `count` copies back to back in one hipGraph on one stream, like a family replay (HIP events)."""
    import ctypes as C

    from hackathon_amd import _lib
    from hackathon_amd.device import Buffer, Event, Stream

    half = max(256, (int(nbytes) // 2 + 255) // 256 * 256)
    src, dst, st = Buffer(half), Buffer(half), Stream()
    ops = (_lib.Op * count)()
    for j in range(count):
        ops[j].kind, ops[j].stream, ops[j].dst, ops[j].src, ops[j].bytes = _lib.OP_COPY, 0, dst.ptr, src.ptr, half
    streams = (C.c_void_p * 1)(st.handle)
    g = C.c_void_p()
    _lib.check(_lib.lib().c3h_program_capture(ops, count, streams, 1, None, 0, C.byref(g)), "c3h_program_capture")
    try:
        _lib.check(_lib.lib().c3h_graph_launch(g.value, st.handle), "c3h_graph_launch")
        e0, e1 = Event(timing=True), Event(timing=True)
        e0.record(st)
        for _ in range(reps):
            _lib.check(_lib.lib().c3h_graph_launch(g.value, st.handle), "c3h_graph_launch")
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps / count
    finally:
        _lib.lib().c3h_graph_destroy(g.value)


def _memory_bound(prog, reps: int) -> dict:
    """Achieved HBM bandwidth of each memory-bound kernel family of the program, beside the
    bandwidth a plain device-to-device copy (hipMemcpyAsync in a graph) reaches moving the same
    bytes per launch, replayed the same way: the practical ceiling for launches of that size."""
    out = {}
    for kind in MEMORY_BOUND:
        idx = prog.launches_of([kind])
        if not idx:
            continue
        repeat = max(1, -(-32 // len(idx)))
        ms = prog.time_subset(idx, reps=reps, repeat=repeat)
        _, nbytes = prog.work(idx)
        gbps = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        per = nbytes / len(idx)
        c_ms = _copy_ms(per, len(idx) * repeat, reps)
        c_gbps = per / (c_ms * 1e-3) / 1e9 if c_ms > 0 else 0.0
        out[kind] = {"launches_per_step": len(idx), "us_per_launch": ms * 1e3 / len(idx),
                     "algorithmic_MB_per_launch": per / 1e6, "achieved_GBps": gbps,
                     "peak_GBps": PEAK["hbm"], "frac_of_hbm_peak": gbps / PEAK["hbm"],
                     "copy_same_bytes_GBps": c_gbps, "frac_of_copy": gbps / c_gbps if c_gbps > 0 else None,
                     "timing": f"hipGraph of the family's launches x{repeat}, HIP events, {reps} replays; copy "
                               f"reference: hipMemcpyAsync D2D of {per / 2e6:.1f} MB, the same count per graph"}
    return out


def _end_to_end(prog, m, units: int, steps: int) -> dict:
    """The program fed from pinned host memory and drained to it, every step."""
    import numpy as np

    from hackathon_amd import _lib
    from hackathon_amd.device import PinnedArray, synchronize

    pin_in = {}
    for n, v in m.inputs.items():
        pa = PinnedArray(v.shape, v.dtype)
        pa.array[...] = v
        pin_in[n] = pa
    pin_out = {n: PinnedArray(a.shape, a.dtype) for n, a in prog.output_arrays.items()}
    feed = {n: (pa, pa.array.nbytes) for n, pa in pin_in.items()}
    h = prog.stream.handle

    def step():
        prog.stage_inputs(feed)
        prog.launch()
        for n, a in prog.output_arrays.items():
            _lib.check(_lib.lib().c3h_memcpy_d2h_async(pin_out[n].ptr, a.ptr, a.nbytes, h), "d2h")

    step()
    prog.stream.synchronize()
    synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    prog.stream.synchronize()
    wall = time.perf_counter() - t0
    in_bytes = sum(pa.array.nbytes for pa in pin_in.values())
    out_bytes = sum(a.nbytes for a in prog.output_arrays.values())
    return {"value": units * steps / wall, "ms_per_step": wall * 1e3 / steps, "steps": steps,
            "h2d_bytes_per_step": in_bytes, "d2h_bytes_per_step": out_bytes,
            "form": "pinned host input -> H2D -> program -> D2H of every output to pinned host, "
                    "serialized on the program stream"}


def _end_to_end_overlapped(name: str, batches: int = 3) -> dict:
    """load_and_infer's streamed pipeline (c35/executor.py:1137-1201 restated over HIP streams): `batches`
    batches from host memory through pinned double buffers, the program, and the logits drained on a copy
    stream in 64 MB pinned chunks into a memory-mapped logits.npy (plus argmax.npy) while the next batch
    runs.  Wall time of the whole run after one warm-up batch (which compiles the plan)."""
    import tempfile

    import numpy as np

    from hackathon_amd import models
    from hackathon_amd.c35.executor import CrossStageReferencePipeline, _stream_compiled
    from hackathon_amd.device import synchronize

    m = models.build(name)
    batch = next(iter(m.inputs.values())).shape[0]
    units = batch * (m.tokens_per_sample if m.unit == "tokens" else 1)
    pipe = CrossStageReferencePipeline(m.graph, m.weights, engine_kind="compiled", precision=m.precision)
    out_name = m.graph.outputs[0].name
    extras = [t.name for t in m.graph.outputs[1:]]
    arrays = {k: np.ascontiguousarray(np.concatenate([v] * batches)) for k, v in m.inputs.items()}
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=shm) as d:
        path = os.path.join(d, "logits.npy")
        _stream_compiled(pipe, m.inputs, batch, batch, out_name, path, extras)
        synchronize()
        t0 = time.perf_counter()
        _stream_compiled(pipe, arrays, batch * batches, batch, out_name, path, extras)
        synchronize()
        wall = time.perf_counter() - t0
    in_bytes = sum(v.nbytes for v in m.inputs.values())
    return {"value": units * batches / wall, "ms_per_batch": wall * 1e3 / batches, "batches": batches,
            "h2d_bytes_per_batch": in_bytes, "output": f"{out_name} (+{', '.join(extras) or 'nothing'}) to a "
            f"memory-mapped .npy under {shm or 'the temp dir'}",
            "form": "load_and_infer's pipeline: pinned double-buffered input, program, logits staged on the "
                    "device and drained on a copy stream while the next batch runs"}


def _blas_info() -> dict:
    """Thread settings and the BLAS NumPy is linked against (BASELINE.md's CPU-baseline plan)."""
    import numpy as np

    info = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    info["affinity_cores"] = len(os.sched_getaffinity(0))
    info["numpy"] = np.__version__
    try:
        cfg = np.show_config(mode="dicts")
        blas = cfg.get("Build Dependencies", {}).get("blas", {})
        info["blas"] = {k: blas.get(k) for k in ("name", "version", "openblas configuration") if blas.get(k)}
    except Exception as exc:  # noqa: BLE001 - informational only
        info["blas"] = f"unavailable: {exc}"
    return info


def _cpu_baseline(name: str, sample: int = 0) -> dict:
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
    b = sample or CPU_SAMPLE[name]
    plan = ExecutionScheduler(m.graph, batch_size=b, precision_policy=PrecisionPolicy(m.precision)).build()
    # the first b samples; a sample larger than the batch repeats the batch (every config is
    # batch-independent), so the timed work is b samples either way
    feed = {k: np.concatenate([v] * -(-b // v.shape[0]))[:b] for k, v in m.inputs.items()}
    assert all(v.shape[0] == b for v in feed.values())
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
                      f"{m.precision} policy rounding emulated in fp32) on {b} samples of the batch (the "
                      f"batch repeated if it has fewer), median of {len(times)} runs ({t:.3f} s each)",
            "threads": _blas_info()}


# -- measured HBM traffic (two rocprofv3 --pmc passes) --------------------------------------------
COPY_BYTES = 1 << 30
TRAFFIC_PROFILE = ROOT / "profiles" / f"{HEADLINE}_conv_traffic.md"


def _traffic_profile(workload: str, label: str) -> Path:
    return ROOT / "profiles" / f"{workload}_{label}_traffic.md"


def _traffic_run(meta_path: str, workload: str = HEADLINE, kinds: str = "", reps: int = 3) -> int:
    """The dispatch stream the FETCH_SIZE and WRITE_SIZE passes count.

    First a plain copy of COPY_BYTES (strided_copy_kernel, 8-byte elements,
    dense): what the counters read for it against the bytes it must move is
    the calibration factor.  Then the workload's launches of `kinds` (default:
    its dominant family) replayed `reps` + 1 times as one hipGraph, as the
    run's last dispatches; their per-launch algorithmic bytes go to
    `meta_path` for the summary."""
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
    m, plan, prog = _prepare(workload)
    kind_list = [k for k in kinds.split(",") if k] or DOMINANT[workload][0]
    label = PROFILE_LABEL[workload] if kind_list == DOMINANT[workload][0] else "_".join(kind_list)
    idx = prog.launches_of(kind_list)
    if not idx:
        raise ValueError(f"{workload} has no launches of kinds {kind_list}")
    prog.time_subset(idx, reps=reps)
    synchronize()
    meta = {"workload": workload, "label": label, "kinds": kind_list, "copy_bytes": COPY_BYTES,
            "copy_dispatches": 3, "replays": reps + 1,
            "launches": [{k: prog.launch_meta[i][k] for k in ("kind", "flops", "bytes")} for i in idx]}
    with open(meta_path, "w") as f:
        json.dump(meta, f, indent=1)
    _log(f"traffic run: {workload} {kind_list}: {len(idx)} launches x {reps + 1} replays, meta -> {meta_path}")
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


def _source_commit() -> str:
    import subprocess

    try:
        return subprocess.run(["git", "-C", str(ROOT), "rev-parse", "--short=12", "HEAD"], capture_output=True,
                              text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        # a copy of the tree without .git (a GPU box): the commit it was taken at, if the caller names it
        return os.environ.get("C3H_SOURCE_COMMIT", "unknown")


def _traffic_summary(fetch_dir: str, write_dir: str, meta_path: str) -> int:
    """Calibrated HBM bytes per launch -> profiles/<workload>_<label>_traffic.md."""
    import numpy as np

    with open(meta_path) as f:
        meta = json.load(f)
    launches = meta["launches"]
    nl, reps = len(launches), meta["replays"]
    out = {}
    names = []
    for counter, run_dir in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _pmc_rows(run_dir, counter)
        copy = [v for k, v in rows if "strided_copy_kernel" in k]
        if len(copy) != meta["copy_dispatches"] or len(rows) < nl * reps:
            raise ValueError(f"{counter}: {len(copy)} copy dispatches (expected {meta['copy_dispatches']}), "
                             f"{len(rows)} dispatches in all (need {nl * reps} for the replays)")
        sub = rows[-nl * reps:]  # the subset graph's replays are the run's last dispatches
        names = [k for k, _ in sub[:nl]]
        factor = meta["copy_bytes"] / (float(np.median(copy)) * 1024.0)
        per = np.asarray([v for _, v in sub]).reshape(reps, nl).mean(axis=0) * 1024.0 * factor
        out[counter] = (factor, float(np.median(copy)), per)
    f_fac, f_copy, fetch = out["FETCH_SIZE"]
    w_fac, w_copy, write = out["WRITE_SIZE"]
    alg = np.asarray([l["bytes"] for l in launches], float)
    traffic = fetch + write
    wl, label = meta["workload"], meta.get("label", "conv")
    kinds = ",".join(meta.get("kinds", DOMINANT[wl][0]))
    dest = _traffic_profile(wl, label)
    lines = [
        f"# {wl}: HBM traffic of the {kinds} launches (rocprofv3 --pmc)", "",
        "Commands (repository root, MI355X box; one counter per pass):", "", "```",
        f"timeout -s KILL 180 rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch -o run -- \\",
        f"    python3 bench.py --traffic-run gpurun_out/traffic_meta_fetch.json --workload {wl} --kinds {kinds}",
        f"timeout -s KILL 180 rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write -o run -- \\",
        f"    python3 bench.py --traffic-run gpurun_out/traffic_meta.json --workload {wl} --kinds {kinds}",
        "python3 bench.py --traffic-summary gpurun_out/pmc_fetch gpurun_out/pmc_write gpurun_out/traffic_meta.json",
        "```", "",
        f"Calibration: a dense copy of {meta['copy_bytes'] / 2**20:.0f} MiB (strided_copy_kernel) reads "
        f"FETCH_SIZE {f_copy:.0f} KiB and WRITE_SIZE {w_copy:.0f} KiB per dispatch; scale factors "
        f"{f_fac:.4f} (fetch) and {w_fac:.4f} (write) turn counter KiB into bytes moved.", "",
        "| launch | kind | kernel | algorithmic MB | fetched MB | written MB | traffic / algorithmic |",
        "|---:|---|---|---:|---:|---:|---:|",
    ]
    for i in range(nl):
        kname = names[i].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:60]
        lines.append(f"| {i} | {launches[i]['kind']} | `{kname}` | {alg[i] / 1e6:.1f} | {fetch[i] / 1e6:.1f} | "
                     f"{write[i] / 1e6:.1f} | {traffic[i] / alg[i]:.2f} |")
    lines += ["", f"Per step: algorithmic {alg.sum() / 1e9:.3f} GB, measured {traffic.sum() / 1e9:.3f} GB "
              f"({traffic.sum() / alg.sum():.2f}x).", "",
              f"traffic_bytes_per_launch = {traffic.mean():.0f}",
              f"algorithmic_bytes_per_launch = {alg.mean():.0f}",
              f"source_commit = {_source_commit()}", ""]
    dest.write_text("\n".join(lines))
    _log(f"wrote {dest}: {traffic.mean() / 1e6:.1f} MB per launch ({traffic.sum() / alg.sum():.2f}x algorithmic)")
    return 0


def _profile_path(workload: str, label: str) -> Path:
    return ROOT / "profiles" / f"{workload}_{label}.md"


def _profile_run(meta_path: str, workload: str = HEADLINE, kinds: str = "", reps: int = 10) -> int:
    """The dispatch stream a `rocprofv3 --kernel-trace --stats` run summarizes.

    The workload's program runs once (realistic buffer contents), then its
    launches of `kinds` (default: the dominant family) are timed exactly as
    the bench line's roofline times them: a hipGraph of just those launches,
    in program order on one stream (so concurrently paired launches run
    serialized), replayed `reps` times between HIP events after one untimed
    replay.  Those replays are the run's last dispatches; the HIP-event time
    and each launch's shape go to `meta_path` for --profile-summary."""
    from hackathon_amd.device import init, synchronize

    init(0)
    m, plan, prog = _prepare(workload)
    kind_list = [k for k in kinds.split(",") if k] or DOMINANT[workload][0]
    label = PROFILE_LABEL[workload] if kind_list == DOMINANT[workload][0] else "_".join(kind_list)
    idx = prog.launches_of(kind_list)
    if not idx:
        raise ValueError(f"{workload} has no launches of kinds {kind_list}")
    prog.run(m.inputs)
    k_ms = prog.time_subset(idx, reps=reps)
    synchronize()
    flops, nbytes = prog.work(idx)
    dtype = DOMINANT[workload][1]
    meta = {"workload": workload, "label": label, "kinds": kind_list, "reps": reps, "event_ms": k_ms,
            "peak": PEAK[dtype], "dtype": dtype, "flops": flops, "bytes": nbytes,
            "launches": [{k: prog.launch_meta[i].get(k) for k in ("kind", "flops", "bytes", "node", "info")}
                         for i in idx]}
    with open(meta_path, "w") as f:
        json.dump(meta, f, indent=1)
    _log(f"profile run: {workload} {kind_list}: {len(idx)} launches, {k_ms:.4f} ms per pass (HIP events, "
         f"{reps} replays) = {flops / (k_ms * 1e-3) / 1e12:.1f} TFLOP/s, meta -> {meta_path}")
    return 0


def _trace_rows(run_dir: str):
    """(kernel name, duration in us) per dispatch, in dispatch order, from a rocprofv3 csv directory."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(run_dir, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *kernel_trace.csv under {run_dir}")
    rows = []
    for path in files:
        with open(path) as f:
            for r in csv.DictReader(f):
                key = int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0)
                rows.append((key, int(r["Start_Timestamp"]), r["Kernel_Name"],
                             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    rows.sort()
    return [(k, d) for _, _, k, d in rows]


def _profile_summary(trace_dir: str, meta_path: str, pmc_dir: str = "") -> int:
    """Per-launch rocprof durations of the --profile-run replays -> profiles/<workload>_<label>.md."""
    import numpy as np

    with open(meta_path) as f:
        meta = json.load(f)
    launches, reps = meta["launches"], meta["reps"]
    nl = len(launches)
    rows = _trace_rows(trace_dir)
    if len(rows) < nl * reps:
        raise ValueError(f"{len(rows)} dispatches in the trace, need {nl * reps} for the timed replays")
    sub = rows[-nl * reps:]
    names = [k for k, _ in sub[:nl]]
    for r in range(reps):
        if [k for k, _ in sub[r * nl:(r + 1) * nl]] != names:
            raise ValueError("the timed replays do not repeat one dispatch sequence")
    us = np.asarray([d for _, d in sub]).reshape(reps, nl).mean(axis=0)
    busy = valu = waves = None
    counters = []
    if pmc_dir:
        import csv
        import glob
        import collections

        d = collections.defaultdict(dict)
        for path in sorted(glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True)):
            with open(path) as f:
                for r in csv.DictReader(f):
                    d[int(r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
        ids = sorted(d)[-nl * reps:]
        counters = sorted({c for i in ids for c in d[i]})

        def per_launch(name):
            return np.asarray([d[i].get(name, 0.0) for i in ids]).reshape(reps, nl).mean(axis=0)

        gr = per_launch("GRBM_GUI_ACTIVE")
        # SQ_VALU_MFMA_BUSY_CYCLES sums the busy cycles of all 1024 SIMDs;
        # GRBM_GUI_ACTIVE sums the dispatch's active cycles over the 8 XCDs:
        # 1024 SIMDs x cycles = 128 x the GRBM sum
        if "SQ_VALU_MFMA_BUSY_CYCLES" in counters:
            busy = per_launch("SQ_VALU_MFMA_BUSY_CYCLES") / np.maximum(128.0 * gr, 1.0)
        # a wave64 VALU instruction occupies its SIMD 4 cycles (more for
        # transcendentals and 64-bit operations): issue share of all SIMD cycles
        if "SQ_INSTS_VALU" in counters:
            valu = per_launch("SQ_INSTS_VALU") * 4.0 / np.maximum(128.0 * gr, 1.0)
        if "SQ_WAVES" in counters:
            waves = per_launch("SQ_WAVES")
    peak, unit = meta["peak"], "TFLOP/s"
    wl, label = meta["workload"], meta["label"]
    kinds = ",".join(meta["kinds"])
    fl = np.asarray([l["flops"] for l in launches], float)
    total_us = float(us.sum())
    frac_table = fl.sum() / (total_us * 1e-6) / 1e12 / peak
    frac_event = fl.sum() / (meta["event_ms"] * 1e-3) / 1e12 / peak
    dest = _profile_path(wl, label)
    lines = [
        f"# {wl}: per-launch rocprof durations of the {kinds} launches", "",
        "The launches bench.py's roofline times, replayed as the bench replays them (one hipGraph of just these",
        "launches, program order, one stream), under the kernel tracer. Commands (repository root, MI355X box):", "",
        "```",
        f"cd /tmp && export TMPDIR=/tmp   # then, from the repository root:",
        f"timeout -s KILL 300 rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_{wl}_{label} -o run -- \\",
        f"    python3 bench.py --profile-run gpurun_out/prof_{wl}_{label}_meta.json --workload {wl} --kinds {kinds}",
    ]
    if pmc_dir:
        lines += [f"timeout -s KILL 120 rocprofv3 --pmc {' '.join(counters)} --output-format csv \\",
                  f"    -d gpurun_out/prof_{wl}_{label}_pmc -o run -- python3 bench.py --profile-run \\",
                  f"    gpurun_out/prof_{wl}_{label}_pmc_meta.json --workload {wl} --kinds {kinds}"]
    lines += [f"python3 bench.py --profile-summary gpurun_out/prof_{wl}_{label} gpurun_out/prof_{wl}_{label}_meta.json"
              + (f" gpurun_out/prof_{wl}_{label}_pmc" if pmc_dir else ""), "```", "",
              f"Each row is the mean over {reps} timed replays. Peak: " +
              (f"{peak:.0f} {unit} ({meta['dtype']} dense MFMA)." if fl.any() else "8 TB/s (HBM3E)."), ""]
    if busy is not None:
        lines += ["MFMA busy %: SQ_VALU_MFMA_BUSY_CYCLES / (128 x GRBM_GUI_ACTIVE), the share of SIMD cycles",
                  "(1024 SIMDs; GRBM_GUI_ACTIVE summed over 8 XCDs) the matrix cores were busy during the launch.", ""]
    if valu is not None:
        lines += ["VALU issue %: SQ_INSTS_VALU x 4 cycles / (128 x GRBM_GUI_ACTIVE), the share of SIMD cycles spent",
                  "issuing VALU instructions (a lower bound: transcendental and 64-bit operations take longer).", ""]
    mem = not fl.any()  # a memory-bound family: bytes, not flops
    nb = np.asarray([l.get("bytes") or 0 for l in launches], float)
    extra = (" MFMA busy % |" if busy is not None else "") + (" VALU issue % |" if valu is not None else "") + \
        (" waves |" if waves is not None else "")
    if mem:
        head = "| launch | node | shape | kernel | us | algorithmic MB | GB/s | % of 8 TB/s |" + extra
    else:
        head = "| launch | node | shape | kernel | us | GFLOP | TFLOP/s | % of peak |" + extra
    lines += [head, "|---:|---|---|---|---:|---:|---:|---:|" + "---:|" * extra.count("|")]
    for i, l in enumerate(launches):
        kname = names[i].replace("(anonymous namespace)::", "").split("(")[0]
        kname = kname.replace("void c3h::gk::", "").replace("void c3h::", "").replace("void ", "")[:70]
        if mem:
            bw = nb[i] / (us[i] * 1e-6) / 1e9 if us[i] > 0 else 0.0
            row = (f"| {i} | {l.get('node') or ''} | {l.get('info') or ''} | `{kname}` | {us[i]:.1f} | "
                   f"{nb[i] / 1e6:.1f} | {bw:.0f} | {100 * bw / 8000.0:.1f} |")
        else:
            t = fl[i] / (us[i] * 1e-6) / 1e12 if us[i] > 0 else 0.0
            row = (f"| {i} | {l.get('node') or ''} | {l.get('info') or ''} | `{kname}` | {us[i]:.1f} | "
                   f"{fl[i] / 1e9:.1f} | {t:.0f} | {100 * t / peak:.1f} |")
        if busy is not None:
            row += f" {100 * busy[i]:.1f} |"
        if valu is not None:
            row += f" {100 * valu[i]:.1f} |"
        if waves is not None:
            row += f" {waves[i]:.0f} |"
        lines.append(row)
    if mem:
        lines += ["", f"Sum of per-launch durations: {total_us:.1f} us for {nb.sum() / 1e6:.1f} MB = "
                  f"{nb.sum() / (total_us * 1e-6) / 1e9:.0f} GB/s, {100 * nb.sum() / (total_us * 1e-6) / 8e12:.1f} % of "
                  f"8 TB/s.", f"HIP events around the same replays: {meta['event_ms'] * 1e3:.1f} us; rocprof sum / event "
                  f"time = {total_us / (meta['event_ms'] * 1e3):.3f}."]
    else:
        lines += ["", f"Sum of per-launch durations: {total_us:.1f} us for {fl.sum() / 1e9:.2f} GFLOP = "
                  f"{fl.sum() / (total_us * 1e-6) / 1e12:.0f} {unit}, {100 * frac_table:.1f} % of peak.",
                  f"HIP events around the same replays (the bench line's kernel_ms_per_step): "
                  f"{meta['event_ms'] * 1e3:.1f} us = {100 * frac_event:.1f} % of peak; rocprof sum / event time = "
                  f"{total_us / (meta['event_ms'] * 1e3):.3f}."]
    lines += [
              "", f"rocprof_us_per_pass = {total_us:.1f}", f"event_us_per_pass = {meta['event_ms'] * 1e3:.1f}",
              f"source_commit = {_source_commit()}", ""]
    dest.write_text("\n".join(lines))
    _log(f"wrote {dest}: {total_us:.1f} us per pass ({100 * frac_table:.1f} % of peak; events "
         f"{meta['event_ms'] * 1e3:.1f} us)")
    return 0


def _committed_traffic():
    """(HBM bytes per dominant launch, source note) from the committed pmc summary, or (None, None)."""
    import re

    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None, None
    m = re.search(r"^traffic_bytes_per_launch = (\d+)$", text, re.M)
    c = re.search(r"^source_commit = (\S+)$", text, re.M)
    src = f"{TRAFFIC_PROFILE.relative_to(ROOT)} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of bench.py " \
          f"--traffic-run, copy-calibrated; tree at commit {c.group(1) if c else 'unrecorded'})"
    return (int(m.group(1)) if m else None), src


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="mlp,resnet18_cifar,resnet18_224,decoder_fp16,decoder_w8a8,decoder_fp4",
                    help="comma-separated workloads to measure (the headline is always included)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-run", metavar="META_JSON",
                    help="dispatch stream for a rocprofv3 --pmc pass (copy calibration + a family's launches)")
    ap.add_argument("--workload", default=HEADLINE, help="workload of --traffic-run")
    ap.add_argument("--kinds", default="", help="launch kinds of --traffic-run (default: the dominant family)")
    ap.add_argument("--traffic-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "META_JSON"),
                    help="turn the two pmc passes into the committed traffic summary (no GPU)")
    ap.add_argument("--profile-run", metavar="META_JSON",
                    help="dispatch stream for rocprofv3 --kernel-trace: a family's launches replayed as the roofline "
                         "times them")
    ap.add_argument("--profile-summary", nargs="+", metavar="DIR",
                    help="TRACE_DIR META_JSON [PMC_DIR]: per-launch table -> profiles/ (no GPU)")
    args = ap.parse_args()
    if args.traffic_summary:
        return _traffic_summary(*args.traffic_summary)
    if args.profile_summary:
        return _profile_summary(*args.profile_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.traffic_run:
        return _traffic_run(args.traffic_run, args.workload, args.kinds)
    if args.profile_run:
        return _profile_run(args.profile_run, args.workload, args.kinds)
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
    head["roofline"]["traffic"], head["roofline"]["traffic_source"] = _committed_traffic()
    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = _cpu_baseline(HEADLINE)
        _log(f"cpu baseline: {cpu['value']:.2f} {cpu['unit']} on {cpu['cores']} threads ({time.time() - t0:.0f}s)")
        for n in names:
            if n == HEADLINE or n not in CPU_SAMPLE_PER_CONFIG:
                continue
            t0 = time.time()
            per[n]["cpu_baseline"] = _cpu_baseline(n, CPU_SAMPLE_PER_CONFIG[n])
            _log(f"cpu baseline {n}: {per[n]['cpu_baseline']['value']:.2f} {per[n]['cpu_baseline']['unit']} "
                 f"({time.time() - t0:.0f}s)")
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
