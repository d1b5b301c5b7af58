"""The five BASELINE configs at their stated sizes, through the exact program bench.py times.

Each test compiles the workload with `workloads.compile_workload` (the c33
passes, the device BN fold, the c34 plan at the BASELINE batch, the compiled
program with its hipGraph and concurrent launch pairs), runs the whole batch
on the GPU, replays it once more (the replay must be bit-identical), and
compares a slice of the batch with the NumPy oracle evaluating the same fused
graph's plan on the same seeded inputs and weights on the CPU.  Every config
is batch-independent (BN folded, no cross-sample op), so the first rows of
the full-batch result must match the oracle run on the first rows alone.

Gates (c35/test_c35.py:88-93 for fp32; north_star for 16-bit and int8):
  fp32 (MLP, CIFAR ResNet)   allclose rtol 1e-3, atol 1e-3 against the oracle
  16-bit (ResNet-224 bf16, decoder fp16)
                             against the oracle with the policy's rounding
                             emulated, and the measured distance to fp32
                             printed; see each test for the asserted bounds
  W8A8                       against the oracle with W8A8 emulated
  W4A16 (config 4's decoder under the "fp4" policy, no BASELINE config)
                             against the oracle with MXFP4 weights emulated
"""

from __future__ import annotations

import time

import numpy as np
import pytest

import gates
from oracle import graph_ref as G

pytestmark = pytest.mark.gpu

# rows of the batch the oracle evaluates (the GPU always runs the full batch)
SLICE = {"mlp": 256, "resnet18_cifar": 8, "resnet18_224": 16, "decoder_fp16": 16, "decoder_w8a8": 1,
         "decoder_fp4": 16}


def _oracle(m, folded, rows: int, policy: str, store=None):
    from hackathon_amd.c32.strategy import PrecisionPolicy
    from hackathon_amd.c34.scheduler import ExecutionScheduler

    plan = ExecutionScheduler(m.graph, batch_size=rows, precision_policy=PrecisionPolicy(m.precision)).build()
    feed = {k: v[:rows] for k, v in m.inputs.items()}
    return G.run_plan(plan, m.graph, {**m.weights, **folded}, feed, policy=policy, store=store)


def _run_full(name: str):
    """Build and compile the workload at its BASELINE size; run the batch twice.

    Returns (model, CPU-folded Conv+BN weights for the oracle, program,
    outputs).  The oracle's fold is taken from the fused graph before the
    device fold rewrites its Conv+BN nodes."""
    import copy

    from hackathon_amd import models
    from hackathon_amd.c33.pipeline import GraphPassPipeline
    from hackathon_amd.workloads import compile_workload

    t0 = time.time()
    m = models.build(name)
    fused = copy.deepcopy(m.graph)
    GraphPassPipeline().run(fused)
    folded = G.fold_conv_bn(fused, m.weights)
    m, plan, prog = compile_workload(name, model=m)
    print(f"{name}: compiled {prog.num_launches} launches ({time.time() - t0:.1f}s), pairs {prog.pairs}", flush=True)
    first = {k: v.get().copy() for k, v in prog.run(m.inputs).items()}
    again = {k: v.get() for k, v in prog.run(m.inputs).items()}
    for k in first:
        np.testing.assert_array_equal(first[k].view(np.uint8), again[k].view(np.uint8))
    return m, folded, prog, first


@pytest.mark.parametrize("name", ["mlp", "resnet18_cifar"])
def test_fullsize_fp32_compiled_and_strict(gpu, name):
    """Configs 1-2 (fp32): the compiled program and the strict planned
    timeline (registry kernels over the c34 arena), both at B=256."""
    from hackathon_amd.c34.scheduler import ExecutionScheduler
    from hackathon_amd.c32.strategy import PrecisionPolicy
    from hackathon_amd.c35.executor import PlannedGraphExecutor
    from hackathon_amd.device import DeviceArray

    m, folded, prog, out = _run_full(name)
    rows = SLICE[name]
    t0 = time.time()
    ref = _oracle(m, folded, rows, "fp32")["logits"]
    print(f"{name}: oracle on {rows} rows {time.time() - t0:.1f}s", flush=True)
    got = out["logits"].reshape((-1,) + ref.shape[1:])[:rows]
    print(f"{name}: compiled max|diff| {float(np.max(np.abs(got - ref))):.3e} (max|logit| "
          f"{float(np.max(np.abs(ref))):.2f})", flush=True)
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3)
    del prog
    from hackathon_amd import models
    from hackathon_amd.c33.pipeline import GraphPassPipeline

    m = models.build(name)  # the strict executor folds Conv+BN itself (X:359-442)
    GraphPassPipeline().run(m.graph)
    ex = PlannedGraphExecutor(m.graph, m.weights)
    batch = next(iter(m.inputs.values())).shape[0]
    splan = ExecutionScheduler(m.graph, batch_size=batch, precision_policy=PrecisionPolicy("fp32")).build()
    feed = {k: DeviceArray.from_host(v) for k, v in m.inputs.items()}
    strict = ex.run_planned(feed, splan)["logits"].get().reshape((-1,) + ref.shape[1:])
    print(f"{name}: strict max|diff| {float(np.max(np.abs(strict[:rows] - ref))):.3e}", flush=True)
    np.testing.assert_allclose(strict[:rows], ref, rtol=1e-3, atol=1e-3)
    # the two GPU paths agree over the whole batch too
    np.testing.assert_allclose(strict, out["logits"].reshape(strict.shape), rtol=1e-3, atol=1e-3)


def _stats(tag: str, got: np.ndarray, ref: np.ndarray) -> dict:
    d = np.abs(got.astype(np.float64) - ref)
    s = {"max_abs": float(d.max()), "rms": float(np.sqrt(np.mean(d * d))), "agree": gates.agree(got, ref),
         "max_ref": float(np.max(np.abs(ref)))}
    print(f"  {tag}: max|diff| {s['max_abs']:.3e}  rms {s['rms']:.3e}  argmax agree {s['agree']:.4f} "
          f"(max|logit| {s['max_ref']:.3f})", flush=True)
    return s


def _check_argmax_output(out: dict) -> None:
    """The ArgMax output equals the first index of the maximum of the program's own logits, every row."""
    if "argmax" not in out:
        return
    lg = out["logits"]
    want = np.argmax(lg.reshape(-1, lg.shape[-1]), axis=-1)
    np.testing.assert_array_equal(out["argmax"].reshape(-1), want)
    print(f"  argmax output == argmax(logits) on all {want.size} rows of [{want.size}, {lg.shape[-1]}]", flush=True)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", ["resnet18_224", "decoder_fp16", "decoder_w8a8", "decoder_fp4"])
def test_fullsize_low_precision(gpu, name):
    """End-to-end gates at full size (the per-launch proof is the teacher-forced test below).

    resnet18_224 (bf16): the logits reach |332| with this config's random-init
      BN, so north_star's absolute 2e-2 is below one bf16 ulp of the output
      scale (2.0 at 332) and cannot be met by any bf16 pipeline: the bf16
      emulation itself, evaluated exactly, is ~1.5 away from fp32.  Gate: the
      program is within one bf16 ulp at the logit scale of the emulation that
      rounds where the program stores bf16, and its argmax equals fp32's on
      every image whose top-2 margin exceeds twice that bound.
    decoder_fp16: north_star as written -- max|logits - fp32| <= 2e-2 -- and
      argmax equal to fp32's on every position whose fp32 top-2 margin exceeds
      2 * 2e-2 (the remaining positions are random-init near-ties).
    decoder_w8a8: int8 codes and accumulators are bit-exact per launch (below);
      end to end, a one-ulp LayerNorm or attention difference moves a few int8
      codes, and twelve quantized layers spread that.  Gate: the program is as
      accurate as the W8A8 definition -- its RMS logit error against fp32 is at
      most 1.1x the emulation's, and its argmax agreement with fp32 at most
      0.02 below the emulation's.
    decoder_fp4: 4-bit weights move the logits away from fp32 by design
      (printed); the program implements the W4A16 definition, so the
      16-bit gate applies against its emulation: max|logits - emulation| <=
      2e-2 and argmax equal to the emulation's wherever its top-2 margin
      exceeds 4e-2.
    """
    m, folded, prog, out = _run_full(name)
    store = prog.rounding_map()
    rows = SLICE[name]
    del prog
    _check_argmax_output(out)
    t0 = time.time()
    refs = _oracle(m, folded, rows, m.precision, store=store)
    ref32 = _oracle(m, folded, rows, "fp32")
    print(f"{name}: oracle on {rows} rows {time.time() - t0:.1f}s", flush=True)
    refs, ref32 = refs["logits"], ref32["logits"]
    got = out["logits"].reshape((-1,) + ref32.shape[1:])[:rows]
    assert np.isfinite(out["logits"]).all()
    vs_emu = _stats(f"{name} vs {m.precision} oracle at the program's rounding points", got, refs)
    vs32 = _stats(f"{name} vs fp32 oracle", got, ref32)
    emu32 = _stats(f"{m.precision} oracle (program's rounding points) vs fp32 oracle", refs, ref32)
    # north_star's literal 16-bit gate (max-abs 2e-2 on logits, >= 99.9 % argmax
    # agreement, both against fp32), reported for the program and for the exact
    # emulation of its rounding points; the asserted gates follow per config.
    print(f"  north_star literal gate, {name}: program max|logits - fp32| {vs32['max_abs']:.4g} "
          f"({'meets' if vs32['max_abs'] <= 2e-2 else 'misses'} 2e-2), argmax agreement {100 * vs32['agree']:.2f} % "
          f"({'meets' if vs32['agree'] >= 0.999 else 'misses'} 99.9 %); the emulation itself: "
          f"{emu32['max_abs']:.4g}, {100 * emu32['agree']:.2f} % (max|logit| {vs32['max_ref']:.1f})", flush=True)
    if name == "resnet18_224":
        bound = gates.ulp_at(vs_emu["max_ref"], "bf16")
        assert vs_emu["max_abs"] <= bound, f"{vs_emu['max_abs']} > one bf16 ulp ({bound}) at the logit scale"
        agree, share = gates.margin_agreement(got, ref32, vs32["max_abs"])
        print(f"  argmax vs fp32 on clear-margin rows: {agree:.4f} ({share:.1%} of rows)", flush=True)
        assert agree == 1.0 and vs32["agree"] == 1.0
    elif name == "decoder_fp16":
        assert vs32["max_abs"] <= 2e-2 and vs_emu["max_abs"] <= 2e-2
        agree, share = gates.margin_agreement(got, ref32, 2e-2)
        print(f"  argmax vs fp32 on positions with margin > 4e-2: {agree:.4f} ({share:.1%} of positions); "
              f"overall {vs32['agree']:.4f}", flush=True)
        assert agree == 1.0
    elif name == "decoder_fp4":
        assert vs_emu["max_abs"] <= 2e-2
        agree, share = gates.margin_agreement(got, refs, 2e-2)
        print(f"  argmax vs the W4A16 emulation on positions with margin > 4e-2: {agree:.4f} ({share:.1%} of "
              f"positions); overall {vs_emu['agree']:.4f}", flush=True)
        assert agree == 1.0
    else:
        assert vs32["rms"] <= 1.1 * emu32["rms"]
        assert vs32["agree"] >= emu32["agree"] - 0.02


def _ordered16(x: np.ndarray, kind: str) -> np.ndarray:
    """Monotone integer code of float32 values that are exact bf16 / fp16 values."""
    if kind == "bf16":
        bits = (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.int32)
    else:
        bits = np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16).astype(np.int32)
    mag = bits & 0x7FFF
    return np.where(bits & 0x8000, -mag, mag)


def _teacher_forced(name: str):
    """Per-value parity at full size.

    The program keeps every value it stores (keep_values); the oracle walks
    the plan for the first rows of the batch, recomputes each node from the
    program's own inputs (teacher forcing, run_plan(teacher=...)) with the
    weights as the program holds them (its device-folded Conv+BN weights,
    rounded to the type each launch reads), and every stored value is
    compared.  Returns {tensor: stats}, {tensor: producing op type} and the
    largest relative difference between the device and CPU Conv+BN folds."""
    import copy

    from hackathon_amd import models
    from hackathon_amd.c32.strategy import PrecisionPolicy
    from hackathon_amd.c33.pipeline import GraphPassPipeline
    from hackathon_amd.c34.scheduler import ExecutionScheduler
    from hackathon_amd.device import DeviceArray
    from hackathon_amd.workloads import compile_workload

    m = models.build(name)
    fused = copy.deepcopy(m.graph)
    GraphPassPipeline().run(fused)
    cpu_fold = G.fold_conv_bn(fused, m.weights)
    m, plan, prog = compile_workload(name, model=m, keep_values=True)
    out = {k: v.get() for k, v in prog.run(m.inputs).items()}
    _check_argmax_output(out)
    gpu_fold = {k: v.get() for k, v in prog.weights_src.items()
                if k.startswith("__c3_folded_") and isinstance(v, DeviceArray)}
    assert set(gpu_fold) == set(cpu_fold)
    fold_rel = _fold_difference(fused, m.weights, gpu_fold, cpu_fold)
    rows = SLICE[name] if name != "mlp" else 64
    store = prog.rounding_map()
    teacher = {n: prog.read_value(n, rows) for n in prog.stored_dtypes()}
    in_registers = set(prog.rounded_in_registers())
    del prog
    stats, ops = {}, {}

    def on_forced(n, ref, got):
        kind = store[n]
        st = {"kind": kind, "size": int(got.size), "max_ref": float(np.max(np.abs(ref))) if ref.size else 0.0}
        if kind in ("int8", "int32", "int64", "u8"):
            st["mismatch"] = int(np.count_nonzero(ref != got))
            st["code_max"] = int(np.max(np.abs(ref.astype(np.int64) - got.astype(np.int64)))) if ref.size else 0
            # codes of a QuantizeLinear fused into its producer's launch (a
            # LayerNorm, or FFN1's GEMM + GELU): the oracle quantizes its own
            # producer output (never stored, so not teacher-forced), which may
            # sit one activation ulp away
            prod_node = m.graph.nodes.get(m.graph.tensor_producer.get(n))
            st["after_fused_producer"] = bool(prod_node is not None and prod_node.inputs and
                                        prod_node.inputs[0] in in_registers)
        else:
            d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
            st["max_abs"] = float(d.max()) if d.size else 0.0
            if kind in ("bf16", "fp16"):
                u = np.abs(_ordered16(got, kind) - _ordered16(G.round_to(ref, kind), kind))
                st["ulp_max"] = int(u.max()) if u.size else 0
                st["frac_gt1"] = float(np.mean(u > 1)) if u.size else 0.0
                st["frac_gt0"] = float(np.mean(u > 0)) if u.size else 0.0
        stats[n] = st
        prod = m.graph.tensor_producer.get(n)
        ops[n] = m.graph.nodes[prod].op_type if prod in m.graph.nodes else "?"

    oplan = ExecutionScheduler(m.graph, batch_size=rows, precision_policy=PrecisionPolicy(m.precision)).build()
    feed = {k: v[:rows] for k, v in m.inputs.items()}
    G.run_plan(oplan, m.graph, {**m.weights, **gpu_fold}, feed, policy=m.precision, store=store, teacher=teacher,
               on_forced=on_forced)
    return stats, ops, fold_rel


def _fold_difference(fused, weights, gpu_fold, cpu_fold) -> float:
    """Largest difference between the device and CPU Conv+BN folds, in units
    of fp32 epsilon (2^-23) relative to the magnitude of what is summed:
    |w * f| for a folded weight, |(b - mean) * f| + |beta| for a folded bias
    (which may cancel to near zero, so its own magnitude is no scale)."""
    worst = 0.0
    for nid, node in fused.nodes.items():
        wn = f"__c3_folded_{nid}_weight__"
        if wn not in cpu_fold:
            continue
        off = int(node.attributes.get("bn_parameter_offset", len(node.inputs)))
        scale, beta, mean, var = (np.asarray(weights[n], np.float64).reshape(-1) for n in node.inputs[off:off + 4])
        f = scale / np.sqrt(var + float(node.attributes.get("bn_epsilon", 1e-5)))
        cb = np.asarray(weights[node.inputs[2]], np.float64).reshape(-1) if off > 2 and node.inputs[2] else 0.0
        w = np.asarray(weights[node.inputs[1]], np.float64)
        wscale = np.abs(w * f.reshape((-1,) + (1,) * (w.ndim - 1)))
        bscale = np.abs((cb - mean) * f) + np.abs(beta)
        bn = f"__c3_folded_{nid}_bias__"
        dw = np.abs(gpu_fold[wn].astype(np.float64) - cpu_fold[wn]) / np.maximum(wscale, 1e-30)
        db = np.abs(gpu_fold[bn].astype(np.float64) - cpu_fold[bn]) / np.maximum(bscale, 1e-30)
        worst = max(worst, float(dw.max()), float(db.max()))
    return worst / 2.0 ** -23


def _summarize(name, stats, ops):
    by = {}
    for n, st in stats.items():
        by.setdefault((ops[n], st["kind"]), []).append((n, st))
    for (op, kind), items in sorted(by.items()):
        if kind in ("int8", "int32", "int64", "u8"):
            worst = max(items, key=lambda t: t[1]["mismatch"])
            fused = sum(1 for t in items if t[1].get("after_fused_producer"))
            print(f"  {name} {op:>25} {kind:>5} x{len(items):3d}: mismatches max {worst[1]['mismatch']} of "
                  f"{worst[1]['size']}, |code diff| <= {worst[1]['code_max']} ({worst[0]}; {fused} quantized inside "
                  f"the producing launch)", flush=True)
        elif kind in ("bf16", "fp16"):
            worst = max(items, key=lambda t: t[1]["max_abs"] / gates.ulp_at(t[1]["max_ref"], kind))
            gt1 = max(t[1]["frac_gt1"] for t in items)
            gt0 = max(t[1]["frac_gt0"] for t in items)
            print(f"  {name} {op:>25} {kind:>5} x{len(items):3d}: max|d| {worst[1]['max_abs']:.3g} = "
                  f"{worst[1]['max_abs'] / gates.ulp_at(worst[1]['max_ref'], kind):.2f} ulp at |ref| "
                  f"{worst[1]['max_ref']:.3g} ({worst[0]}); elements >1 own ulp {gt1:.1e}, >0 {gt0:.1e}", flush=True)
        else:
            worst = max(items, key=lambda t: t[1]["max_abs"] / max(t[1]["max_ref"], 1e-30))
            print(f"  {name} {op:>25} {kind:>5} x{len(items):3d}: max |d| {worst[1]['max_abs']:.3e} "
                  f"(|ref| {worst[1]['max_ref']:.3g}; {worst[0]})", flush=True)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", ["mlp", "resnet18_cifar", "resnet18_224", "decoder_fp16", "decoder_w8a8",
                                  "decoder_fp4"])
def test_fullsize_per_value_teacher_forced(gpu, name):
    """Every value the full-size program stores, against the oracle's node
    recomputed from the program's own inputs (no error carried between nodes):
      int8 (QuantizeLinear codes)            bit-exact; codes quantized inside the
                                             producing launch (W8A8: LayerNorm, FFN1
                                             GEMM + GELU) within one code on at most
                                             1e-4 of elements, since the oracle
                                             quantizes its own producer output (one
                                             activation ulp at most, above)
      bf16 / fp16                            within one ulp at the tensor's
                                             largest magnitude, and at most
                                             0.1 % of elements more than one
                                             ulp of their own value away
                                             (attention context excepted: the
                                             flash kernel rounds the
                                             probabilities to 16 bits before
                                             P.V, so its error follows the
                                             row's scale, not each element's)
      fp32                                   within 1e-5 of the tensor's largest magnitude
    and the device Conv+BN fold within 4 fp32 epsilons of the CPU fold, relative
    to the magnitude of the terms each folded value sums (a few roundings)."""
    stats, ops, fold_rel = _teacher_forced(name)
    print(f"{name}: {len(stats)} stored values checked; device vs CPU Conv+BN fold within {fold_rel:.2f} fp32 eps",
          flush=True)
    _summarize(name, stats, ops)
    assert stats
    assert fold_rel <= 4.0
    for n, st in stats.items():
        kind = st["kind"]
        if kind in ("int8", "int32", "int64", "u8"):
            if st.get("after_fused_producer"):
                assert st["code_max"] <= 1 and st["mismatch"] <= 1e-4 * st["size"], (n, st)
            else:
                assert st["mismatch"] == 0, (n, st)
        elif kind in ("bf16", "fp16"):
            assert st["max_abs"] <= gates.ulp_at(st["max_ref"], kind), (n, ops[n], st)
            if ops[n] != "MatMul":
                assert st["frac_gt1"] <= 1e-3, (n, ops[n], st)
        else:
            assert st["max_abs"] <= 1e-5 * max(st["max_ref"], 1.0), (n, ops[n], st)


@pytest.mark.parametrize("layer", ["layer0.qkv", "layer0.ffn1", "layer5.ffn2", "lm_head"])
def test_fullsize_qlinear_matmul_bit_exact(gpu, layer):
    """One QLinearMatMul of the real W8A8 model at its full shape
    ([16*1024, K] x the model's int8 weight), fed int8 activations: the int32
    accumulators (qgemm mode 0) and the requantized int8 output with the
    model's own scales (mode 1, the QLinearMatMul node) equal the exact
    integer oracle bit for bit.  The LM head (N = 32000) is checked on 1024
    rows spread over the batch; the other layers on every row."""
    from hackathon_amd import models
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray
    from oracle import registry_ref as R

    m = models.build("decoder_w8a8")
    wq = m.weights[f"{layer}.weight_q"]                      # [K, N] int8
    sb = m.weights[f"{layer}.weight_scale"].astype(np.float32)
    sa = np.float32(m.weights[f"{layer}.act_scale"])
    sy = np.float32(m.weights[f"{layer}.out_scale"])
    k, n = wq.shape
    rows = 16 * 1024
    rng = np.random.default_rng(k + n)
    # activation codes as QuantizeLinear produces them: rounded, saturated, both tails present
    a = np.clip(np.rint(rng.standard_normal((rows, k)) * 40.0), -128, 127).astype(np.int8)
    ad, btd, sbd = DeviceArray.from_host(a), DeviceArray.from_host(np.ascontiguousarray(wq.T)), \
        DeviceArray.from_host(sb)
    acc_d = DeviceArray.empty((rows, n), np.int32)
    y_d = DeviceArray.empty((rows, n), np.int8)
    print(f"qlinear {layer}: {rows}x{n}x{k}", flush=True)
    E.qgemm(ad, btd, acc_d, rows, n, k, mode=0)
    E.qgemm(ad, btd, y_d, rows, n, k, mode=1, a_scale=float(sa), b_scale=sbd, y_scale=float(sy))
    acc, y = acc_d.get(), y_d.get()
    check = np.arange(rows) if n <= 4096 else np.unique(np.linspace(0, rows - 1, 1024).astype(np.int64))
    for lo in range(0, len(check), 4096):
        r = check[lo:lo + 4096]
        want = R.qlinear_matmul_acc(a[r], 0, wq, np.zeros(n, np.int8))
        np.testing.assert_array_equal(acc[r], want)
        np.testing.assert_array_equal(y[r], R.requantize(want, sa, sb, sy, 0))
    sat = float(np.mean(np.abs(y[check].astype(np.int32)) == 127))
    print(f"  bit-exact on {len(check)} rows; |acc| max {int(np.abs(acc[check]).max())}, "
          f"saturated codes {sat:.3%}", flush=True)
