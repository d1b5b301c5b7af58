"""Planned execution on the MI355X (counterpart of c35/executor.py).

`PlannedGraphExecutor.run_planned(feed, plan)` interprets the C3.4 timeline
exactly like the reference (c35/executor.py:723-903): ALLOC/FREE are
bookkeeping, H2D/D2H are async copies on the transfer's stream,
EVENT_RECORD/EVENT_WAIT map to hipEventRecord / hipStreamWaitEvent, and each
KERNEL action calls the registry kernel named by the step
(`kernel_registry.lookup(name)(inputs, outputs, params, tuning)`) with
full-capacity fp32 arena views as outputs.  The arena is one hipMalloc slab
per plan, streams are persistent non-blocking hipStream_t, events are
hipEvent_t per plan, and model tensors stay resident across batches.

Fixed relative to the reference: pinned staging for D2H is allocated once
per plan and reused (X:854), and validating a plan is O(n log n).

`CrossStageReferencePipeline` and `load_and_infer` keep the reference's
orchestration (X:906-1265).  `load_and_infer(..., engine="compiled")`
executes the same plan through `compiled.CompiledPlan` (launch grouping,
fused epilogues, channels-last activations, hipGraph replay) instead.
"""

from __future__ import annotations

import copy
import json
import math
import os
import time
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import _lib
from ..c3common.ir.graph import Graph, Node, ONNSType
from ..c34.execution_plan import ExecutionPlan
from ..device import Buffer, DeviceArray, Event, Stream, current_stream, init, using_stream
from . import engine


# -- weights ---------------------------------------------------------------------------------------
def load_weights(source) -> Tuple[Dict[str, Any], Dict[str, Any]]:
    """(initializers, constants) host arrays from a weights dict or an .onnx path."""
    if isinstance(source, dict):
        return dict(source), {}
    from ..onnx_io import read_initializers_and_constants

    return read_initializers_and_constants(str(source))


class GraphExecutor:
    """Node-by-node execution (X:91-321) through the HIP engine."""

    def __init__(self, graph: Graph, weights) -> None:
        init()
        self.graph = graph
        host_w, host_c = load_weights(weights)
        self.weights = {k: DeviceArray.from_host(np.asarray(v)) for k, v in host_w.items()}
        self.constants = {k: DeviceArray.from_host(np.asarray(v)) for k, v in host_c.items()}
        self.values: Dict[str, DeviceArray] = {}

    def run(self, feed_dict: Dict[str, DeviceArray]) -> Dict[str, DeviceArray]:
        self.values = {**self.weights, **self.constants, **feed_dict}
        for nid in self.graph.node_order:
            node = self.graph.nodes.get(nid)
            if node is not None:
                self._execute_node(node)
        out = {}
        for t in self.graph.outputs:
            if t.name not in self.values:
                raise KeyError(f"Graph output '{t.name}' not found in computed values")
            out[t.name] = self.values[t.name]
        return out

    def _execute_node(self, node: Node) -> None:
        if node.op_type == "Constant":
            for o in node.outputs:
                if o and o not in self.values:
                    raise KeyError(f"Constant node '{node.id}' output '{o}' not pre-loaded")
            return
        inputs = []
        for name in node.inputs:
            if not name:
                inputs.append(None)
            elif name not in self.values:
                raise KeyError(f"Node '{node.id}' ({node.op_type}) requires input '{name}' which is not available")
            else:
                inputs.append(self.values[name])
        attrs = dict(node.attributes)
        if node.op_type in ("Split", "LayerNormalization"):
            attrs["_num_outputs"] = len(node.outputs)
        try:
            result = engine.execute_op(node.op_type, inputs, attrs)
        except Exception as exc:
            raise RuntimeError(f"Failed to execute node '{node.id}' ({node.op_type}): {exc}") from exc
        if isinstance(result, list):
            for o, r in zip(node.outputs, result):
                if o:
                    self.values[o] = r
        else:
            for o in node.outputs:
                if o:
                    self.values[o] = result


def fold_conv_batchnorm(graph: Graph, host_weights: Dict[str, Any], stream=None) -> Dict[str, DeviceArray]:
    """Fold every unfolded FusedConv2dBatchNorm on the device (X:359-442).

    Returns {folded name: device array}; rewrites the node to consume
    (x, folded weight, folded bias) with bn_folded=True.
    """
    folded: Dict[str, DeviceArray] = {}
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if node is None or node.op_type != "FusedConv2dBatchNorm" or node.attributes.get("bn_folded"):
            continue
        off = int(node.attributes.get("bn_parameter_offset", len(node.inputs)))
        conv_in, bn_in = list(node.inputs[:off]), list(node.inputs[off:off + 4])
        if len(conv_in) < 2 or len(bn_in) != 4:
            raise ValueError(f"Fused Conv+BN node '{nid}' has an invalid parameter ABI")
        missing = [n for n in [conv_in[1], *bn_in] if n not in host_weights]
        if missing:
            raise ValueError(f"Fused Conv+BN node '{nid}' cannot resolve initializers: {missing}")
        w = np.asarray(host_weights[conv_in[1]], np.float32)
        params = [np.asarray(host_weights[n], np.float32).reshape(-1) for n in bn_in]
        if any(p.size != w.shape[0] for p in params):
            raise ValueError(f"Fused Conv+BN node '{nid}' parameter/channel mismatch")
        dw = DeviceArray.from_host(w)
        ds = [DeviceArray.from_host(p) for p in params]
        cb = None
        if len(conv_in) >= 3 and conv_in[2]:
            if conv_in[2] not in host_weights:
                raise ValueError(f"Fused Conv+BN node '{nid}' cannot resolve Conv bias '{conv_in[2]}'")
            cb = DeviceArray.from_host(np.asarray(host_weights[conv_in[2]], np.float32).reshape(-1))
        w_out = DeviceArray.empty(w.shape, np.float32)
        b_out = DeviceArray.empty((w.shape[0],), np.float32)
        a = _lib.BnFoldArgs()
        a.w, a.conv_bias = dw.ptr, cb.ptr if cb is not None else None
        a.scale, a.bias, a.mean, a.var = ds[0].ptr, ds[1].ptr, ds[2].ptr, ds[3].ptr
        a.w_out, a.b_out = w_out.ptr, b_out.ptr
        a.out_channels, a.per_channel = w.shape[0], int(np.prod(w.shape[1:]))
        a.epsilon = float(node.attributes.get("bn_epsilon", 1e-5))
        _lib.launch(a, stream)
        wn, bn = f"__c3_folded_{nid}_weight__", f"__c3_folded_{nid}_bias__"
        folded[wn], folded[bn] = w_out, b_out
        for name, arr in ((wn, w_out), (bn, b_out)):
            t = graph.register_tensor(name, dtype=ONNSType.FLOAT, shape=list(arr.shape), is_initializer=True)
            graph.initializers[name] = t
            graph.tensor_producer[name] = "INITIALIZER"
        graph.replace_node_inputs(nid, list(node.inputs), [conv_in[0], wn, bn])
        node.attributes.update({"bn_folded": True, "bn_parameter_offset": 3, "folded_weight": wn,
                                "folded_bias": bn})
    graph.validate()
    return folded


class PlannedGraphExecutor(GraphExecutor):
    """Timeline interpreter over one slab, HIP streams and HIP events."""

    def __init__(self, graph: Graph, weights) -> None:
        init()
        self.graph = graph
        self.host_weights, self.host_constants = load_weights(weights)
        self._preplanned_device_tensors: set = set()
        folded = fold_conv_batchnorm(graph, self.host_weights)
        self.host_weights.update(folded)
        self._preplanned_device_tensors.update(folded)
        self.weights: Dict[str, Any] = {}
        self.constants: Dict[str, Any] = {}
        self.values: Dict[str, DeviceArray] = {}
        self.last_execution_trace: List[Dict[str, Any]] = []
        self.last_host_outputs: Dict[str, np.ndarray] = {}
        self.memory_trace: List[Dict[str, Any]] = []
        self._arena_cache: Dict[int, Tuple[ExecutionPlan, DeviceArray]] = {}
        self._pinned_cache: Dict[int, Dict[str, Tuple[int, int]]] = {}
        self._resident_model_tensors: Dict[str, DeviceArray] = {}
        self._streams: Dict[int, Stream] = {}
        self._events_by_plan: Dict[int, Tuple[ExecutionPlan, Dict[str, Event]]] = {}
        self._validated_plans: Dict[int, ExecutionPlan] = {}
        self._stream_objects_created = 0
        self._event_objects_created = 0
        self._planned_runs = 0
        self._memory_trace_dropped = 0

    @staticmethod
    def _allocation_view(arena: DeviceArray, allocation, shape, dtype) -> DeviceArray:
        dtype = np.dtype(dtype)
        need = math.prod(int(d) for d in shape) * dtype.itemsize
        cap = allocation.capacity_bytes or allocation.size_bytes
        if need > cap:
            raise ValueError(f"Tensor '{allocation.tensor_name}' requires {need} bytes, planned capacity is {cap}")
        return DeviceArray(arena.ptr + allocation.offset_bytes, tuple(shape), dtype, arena.owner)

    def _runtime_resources(self, plan: ExecutionPlan):
        ids = sorted({a.stream_id for a in plan.timeline if a.kind not in ("ALLOC", "FREE")})
        for sid in ids:
            if sid not in self._streams:
                self._streams[sid] = Stream()
                self._stream_objects_created += 1
        cached = self._events_by_plan.get(id(plan))
        if cached is None or cached[0] is not plan:
            events = {e.event_id: Event() for e in plan.events}
            self._events_by_plan[id(plan)] = (plan, events)
            self._event_objects_created += len(events)
        else:
            events = cached[1]
        return {sid: self._streams[sid] for sid in ids}, events

    def runtime_resource_stats(self) -> Dict[str, int]:
        return {"planned_runs": self._planned_runs, "stream_objects_created": self._stream_objects_created,
                "stream_objects_active": len(self._streams), "event_objects_created": self._event_objects_created,
                "event_plan_count": len(self._events_by_plan), "memory_trace_records": len(self.memory_trace),
                "memory_trace_dropped": self._memory_trace_dropped}

    def _arena(self, plan: ExecutionPlan) -> DeviceArray:
        need = max(1, plan.pool_stats.peak_reserved_bytes)
        cached = self._arena_cache.get(id(plan))
        if cached is None or cached[0] is not plan or cached[1].nbytes < need:
            buf = Buffer(need)
            self._arena_cache[id(plan)] = (plan, DeviceArray(buf.ptr, (need,), np.uint8, buf))
        return self._arena_cache[id(plan)][1]

    def _copy_h2d(self, source: Any, dest: DeviceArray, stream: Stream) -> None:
        if isinstance(source, DeviceArray):
            with using_stream(stream):
                engine.cast_into(source.reshape(dest.shape) if source.size == dest.size else source, dest)
            return
        host = np.ascontiguousarray(np.asarray(source, dtype=dest.dtype)).reshape(dest.shape)
        dest.copy_from_host(host, stream.handle)
        stream.synchronize()  # pageable source: keep the host buffer alive until the copy completes

    def _execute_planned_node(self, node: Node, step, arena: DeviceArray, allocations: Dict[str, Any]) -> None:
        from ..c32.kernel_registry import lookup

        if step.kernel_name == "constant":
            return
        inputs = []
        for name in step.logical_inputs:
            if not name:
                inputs.append(None)
            elif name not in self.values:
                raise KeyError(f"Kernel '{step.kernel_name}' (node '{step.node_id}') requires unavailable input '{name}'")
            else:
                inputs.append(self.values[name])
        outputs = []
        for name in step.logical_outputs:
            if not name:
                continue
            aid = step.outputs.get(name)
            if aid is None or aid not in allocations:
                raise KeyError(f"Kernel '{step.kernel_name}' output '{name}' has no allocation")
            a = allocations[aid]
            cap = a.capacity_bytes or a.size_bytes
            outputs.append(DeviceArray(arena.ptr + a.offset_bytes, (cap // 4,), np.float32, arena.owner))
        prof = step.precision_profile or {}
        if prof.get("compute_dtype", "fp32") not in ("fp32",) and step.kernel_name not in (
                "quantize_linear", "qlinear_matmul", "dequantize_linear"):
            raise RuntimeError(f"precision {prof.get('compute_dtype')} plans run through the compiled engine")
        lookup(step.kernel_name)(inputs, outputs, dict(step.operator_params), step.tuning_params)
        for name, view in zip([n for n in step.logical_outputs if n], outputs):
            t = self.graph.tensors.get(name)
            if t is not None and t.shape:
                shape = self._resolve_shape_from_graph(t.shape, view.size)
                if shape is not None and math.prod(shape) == view.size:
                    view = view.reshape(shape)
            self.values[name] = view

    @staticmethod
    def _resolve_shape_from_graph(shape: List[Any], total: int) -> Optional[Tuple[int, ...]]:
        """Graph shape with symbolic dims solved from the element count (X:606-671)."""
        known, resolved = 1, []
        for d in shape:
            if d is None:
                resolved.append(-1)
                continue
            try:
                v = int(d)
            except (TypeError, ValueError):
                if isinstance(d, str) and (d.lower() in ("n", "batch", "b") or d.startswith("unk_")):
                    resolved.append(-1)
                    continue
                return None
            if v > 0:
                known *= v
                resolved.append(v)
            elif v == -1:
                resolved.append(-1)
            else:
                return None
        if known <= 0:
            return (total,)
        sym = resolved.count(-1)
        if sym == 0:
            return tuple(resolved)
        if total % known:
            return None
        rem = total // known
        if sym == 1:
            return tuple(rem if d == -1 else d for d in resolved)
        root = round(rem ** (1.0 / sym))
        if root > 0 and root ** sym == rem:
            return tuple(root if d == -1 else d for d in resolved)
        out, first = [], True
        for d in resolved:
            if d == -1:
                out.append(rem if first else 1)
                first = False
            else:
                out.append(d)
        return tuple(out)

    def _pinned(self, plan: ExecutionPlan, name: str, nbytes: int) -> int:
        cache = self._pinned_cache.setdefault(id(plan), {})
        hit = cache.get(name)
        if hit is None or hit[1] < nbytes:
            import ctypes
            ptr = ctypes.c_void_p()
            _lib.check(_lib.lib().c3h_host_alloc(ctypes.byref(ptr), max(nbytes, 1)), "c3h_host_alloc")
            cache[name] = (int(ptr.value), nbytes)
            hit = cache[name]
        return hit[0]

    def weight_sources(self) -> Dict[str, Any]:
        """Every model tensor by name: host payloads plus the device-resident ones.

        Folded Conv+BN parameters leave `host_weights` once a planned run has
        made them resident; the compiled engine needs them either way.
        """
        return {**self.host_weights, **self._resident_model_tensors}

    def run_planned(self, feed_dict: Dict[str, Any], plan: ExecutionPlan) -> Dict[str, DeviceArray]:
        # The structural checks run on the first batch a plan object sees, not
        # on every batch as c35/executor.py:728 does; a plan edited after its
        # first run is the caller's to re-validate.  The feed and graph checks
        # below still run per batch.
        if self._validated_plans.get(id(plan)) is not plan:
            issues = plan.validate()
            if issues:
                raise ValueError("C3.4 execution plan is invalid: " + "; ".join(issues[:10]))
            self._validated_plans[id(plan)] = plan
        counts = {int(np.shape(a)[0]) for a in feed_dict.values() if len(np.shape(a)) > 0}
        if len(counts) != 1:
            raise ValueError("Planned execution requires equal input batch sizes")
        if plan.batch_size != next(iter(counts)):
            raise ValueError(f"Plan batch size {plan.batch_size} does not match feed batch size {next(iter(counts))}")
        seen = {s.node_id for s in plan.kernel_steps}
        nodes = set(self.graph.nodes)
        if seen != nodes:
            raise ValueError("C3.4 plan/optimized-graph mismatch: "
                             f"missing_nodes={sorted(nodes - seen)[:10]}, unexpected_nodes={sorted(seen - nodes)[:10]}")
        if not plan.timeline:
            raise ValueError("C3.4 execution plan has no executable timeline")
        allocations = {a.alloc_id: a for a in plan.allocations}
        arena = self._arena(plan)
        streams, events = self._runtime_resources(plan)
        newly_resident: Dict[str, DeviceArray] = {}
        self.values.clear()
        self.last_execution_trace.clear()
        self.last_host_outputs.clear()
        for act in plan.timeline:
            entry = {"step_index": act.step_index, "kind": act.kind, "stream_id": act.stream_id,
                     "tensor_name": act.tensor_name, "event_id": act.event_id, "status": "executed"}
            self.last_execution_trace.append(entry)
            if act.kind == "ALLOC":
                continue
            if act.kind == "FREE":
                if act.tensor_name is not None:
                    self.values.pop(act.tensor_name, None)
                continue
            stream = streams[act.stream_id]
            if act.kind == "EVENT_WAIT":
                stream.wait_event(events[act.event_id])
            elif act.kind == "EVENT_RECORD":
                events[act.event_id].record(stream)
            elif act.kind == "H2D":
                t = plan.transfers[act.ref_index]
                alloc = allocations[t.alloc_id]
                is_model = t.tensor_name in plan.weight_slots
                resident = self._resident_model_tensors.get(t.tensor_name) or newly_resident.get(t.tensor_name)
                if is_model and resident is not None:
                    dest = self._allocation_view(arena, alloc, resident.shape, resident.dtype)
                    entry["status"] = "resident"
                    if resident.ptr != dest.ptr:
                        with using_stream(stream):
                            engine.copy_into(resident, dest)
                else:
                    if t.tensor_name in feed_dict:
                        src = feed_dict[t.tensor_name]
                    elif t.tensor_name in self.host_weights:
                        src = self.host_weights[t.tensor_name]
                    elif t.tensor_name in self.host_constants:
                        src = self.host_constants[t.tensor_name]
                    else:
                        raise KeyError(f"No H2D source for '{t.tensor_name}'")
                    dtype = src.dtype if isinstance(src, DeviceArray) else np.asarray(src).dtype
                    dest = self._allocation_view(arena, alloc, np.shape(src) if not isinstance(src, DeviceArray)
                                                 else src.shape, dtype)
                    self._copy_h2d(src, dest, stream)
                    if is_model:
                        newly_resident[t.tensor_name] = dest
                self.values[t.tensor_name] = dest
            elif act.kind == "KERNEL":
                step = plan.kernel_steps[act.ref_index]
                with using_stream(stream):
                    self._execute_planned_node(self.graph.nodes[step.node_id], step, arena, allocations)
            elif act.kind == "D2H":
                t = plan.transfers[act.ref_index]
                if t.tensor_name not in self.values:
                    raise KeyError(f"D2H source '{t.tensor_name}' is unavailable")
                src = self.values[t.tensor_name]
                host = self._pinned(plan, t.tensor_name, src.nbytes)
                _lib.check(_lib.lib().c3h_memcpy_d2h_async(host, src.ptr, src.nbytes, stream.handle), "d2h")
                self.last_host_outputs[t.tensor_name] = (host, src.shape, src.dtype)
            else:
                raise ValueError(f"Unsupported timeline action: {act.kind}")
        for s in streams.values():
            s.synchronize()
        engine.check_gather_errors()
        self._resident_model_tensors.update(newly_resident)
        for name in self._preplanned_device_tensors & newly_resident.keys():
            self.host_weights.pop(name, None)
        self._preplanned_device_tensors.difference_update(newly_resident)
        self._planned_runs += 1
        record = {"run_index": self._planned_runs, "batch_size": plan.batch_size,
                  "plan_arena_bytes": max(1, plan.pool_stats.peak_reserved_bytes), "logical_stream_count": len(streams)}
        if len(self.memory_trace) < 64:
            self.memory_trace.append(record)
        else:
            self.memory_trace[-1] = record
            self._memory_trace_dropped += 1
        out = {}
        for t in self.graph.outputs:
            if t.name not in self.values:
                raise KeyError(f"Planned graph did not produce '{t.name}'")
            out[t.name] = self.values[t.name]
        return out

    def host_output(self, name: str) -> np.ndarray:
        """The D2H copy of a graph output from the last run (pinned buffer)."""
        import ctypes

        ptr, shape, dtype = self.last_host_outputs[name]
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        raw = (ctypes.c_uint8 * n).from_address(ptr)
        return np.frombuffer(raw, dtype=dtype).reshape(shape).copy()


class CrossStageReferencePipeline:
    """Fuse (C3.3) -> plan per batch size (C3.4) -> execute (C3.5) (X:906-994)."""

    def __init__(self, graph: Graph, weights, qualify_optimizations: bool = False, engine_kind: str = "planned",
                 precision: str = "fp32") -> None:
        from ..c33.pipeline import GraphPassPipeline

        baseline = copy.deepcopy(graph)
        self.graph = graph
        self.fusion_result = GraphPassPipeline().run(self.graph)
        if not self.fusion_result["Fusion"]["stats"]["validation_passed"]:
            raise ValueError("C3.3 produced an invalid optimized graph")
        self.baseline_executor = GraphExecutor(baseline, weights) if qualify_optimizations else None
        self.optimized_executor = PlannedGraphExecutor(self.graph, weights)
        self.engine_kind = engine_kind
        self.precision = precision
        self._plan_cache: Dict[int, ExecutionPlan] = {}
        self._compiled: Dict[int, Any] = {}
        self._qualified = not qualify_optimizations
        self.qualification_max_abs_diff: Optional[float] = None
        self.last_plan: Optional[ExecutionPlan] = None

    def _plan_for_batch(self, batch_size: int) -> ExecutionPlan:
        from ..c32.strategy import PrecisionPolicy
        from ..c34.scheduler import ExecutionScheduler

        if batch_size not in self._plan_cache:
            plan = ExecutionScheduler(self.graph, batch_size=batch_size,
                                      precision_policy=PrecisionPolicy(self.precision)).build()
            issues = plan.validate()
            if issues:
                raise ValueError("C3.4 rejected before execution: " + "; ".join(issues[:10]))
            self._plan_cache[batch_size] = plan
        return self._plan_cache[batch_size]

    def compiled_for_batch(self, batch_size: int):
        from .compiled import CompiledPlan

        if batch_size not in self._compiled:
            plan = self._plan_for_batch(batch_size)
            ex = self.optimized_executor
            self._compiled[batch_size] = CompiledPlan(self.graph, plan, ex.weight_sources(), ex.host_constants,
                                                      policy=self.precision)
        return self._compiled[batch_size]

    def run(self, feed_dict: Dict[str, Any]) -> Dict[str, DeviceArray]:
        counts = {int(np.shape(a)[0]) for a in feed_dict.values() if len(np.shape(a)) > 0}
        if len(counts) != 1:
            raise ValueError("All graph inputs must have the same batch dimension")
        batch = next(iter(counts))
        plan = self._plan_for_batch(batch)
        self.last_plan = plan
        if self.engine_kind == "compiled":
            optimized = self.compiled_for_batch(batch).run(feed_dict)
        else:
            optimized = self.optimized_executor.run_planned(feed_dict, plan)
        if not self._qualified:
            baseline = self.baseline_executor.run({k: v if isinstance(v, DeviceArray) else DeviceArray.from_host(v)
                                                   for k, v in feed_dict.items()})
            max_diff = 0.0
            for name, expected in baseline.items():
                if name not in optimized:
                    raise KeyError(f"Optimized graph did not produce '{name}'")
                got = optimized[name].get().astype(np.float32)
                exp = expected.get().astype(np.float32)
                if got.shape != exp.shape:
                    raise ValueError(f"Optimized output '{name}' shape {got.shape} != baseline {exp.shape}")
                if got.size:
                    max_diff = max(max_diff, float(np.max(np.abs(got - exp))))
                if not np.allclose(got, exp, rtol=1e-3, atol=1e-3):
                    raise ValueError(f"C3.3 numerical qualification failed for '{name}': max_abs_diff={max_diff:.6e}")
            self.qualification_max_abs_diff = max_diff
            self._qualified = True
        return optimized


def _check_output(out: DeviceArray, out_name: str, tail: Optional[Tuple[int, ...]]) -> Tuple[int, ...]:
    if out.dtype != np.float32:
        raise ValueError(f"Output '{out_name}' must be float32, got {out.dtype}")
    if tail is not None and out.shape[1:] != tail:
        raise ValueError(f"Output '{out_name}' changed non-batch shape from {tail} to {out.shape[1:]}")
    return out.shape[1:]


def _extra_path(out_path: str, name: str) -> str:
    """File of a graph output after the first: <name>.npy beside logits.npy."""
    return os.path.join(os.path.dirname(out_path), f"{name}.npy")


def _run_planned_batches(pipeline, arrays, total, batch, out_name, out_path,
                         extras: Sequence[str] = ()) -> Tuple[int, ...]:
    """Strict path: one batch at a time, logits gathered on the device (X:1137-1201).
    Further graph outputs (`extras`, e.g. an int64 ArgMax) are gathered on
    the host and saved as <name>.npy."""
    final: Optional[DeviceArray] = None
    extra_host: Dict[str, list] = {n: [] for n in extras}
    for start in range(0, total, batch):
        end = min(start + batch, total)
        outs = pipeline.run({name: DeviceArray.from_host(arr[start:end]) for name, arr in arrays.items()})
        out = outs[out_name]
        tail = _check_output(out, out_name, final.shape[1:] if final is not None else None)
        if final is None:
            final = DeviceArray.empty((total,) + tail, np.float32)
        engine.copy_into(out, final.split_axis0(start, end))
        for n in extras:
            extra_host[n].append(outs[n].get())
    if final is None:
        raise RuntimeError("Inference produced no output batches")
    result = final.get()
    if not np.all(np.isfinite(result)):
        raise ValueError("Output contains non-finite values (NaN or Inf)")
    np.save(out_path, result)
    for n in extras:
        np.save(_extra_path(out_path, n), np.concatenate(extra_host[n], axis=0))
    return result.shape


_CHUNK_BYTES = 64 << 20
_COPY_THREADS = 8
_POOL = None


def _copy_pool():
    """Host threads for the streamed pipeline's large host copies (NumPy copies release the GIL)."""
    global _POOL
    if _POOL is None:
        import concurrent.futures as cf

        _POOL = cf.ThreadPoolExecutor(max_workers=_COPY_THREADS, thread_name_prefix="c3h-copy")
    return _POOL


class _NpyWriter:
    """A .npy file written by positioned writes from pinned chunks: the header
    first (NumPy's format), the data region sized up front, then pwrite of
    each piece from the copy threads -- no memory map whose pages would fault
    in one at a time."""

    def __init__(self, path: str, dtype, shape: Tuple[int, ...]) -> None:
        self.dtype = np.dtype(dtype)
        with open(path, "wb") as f:
            np.lib.format.write_array_header_1_0(f, {"descr": np.lib.format.dtype_to_descr(self.dtype),
                                                     "fortran_order": False, "shape": tuple(shape)})
            self.offset = f.tell()
            f.truncate(self.offset + math.prod(shape) * self.dtype.itemsize)
        self.fd = os.open(path, os.O_WRONLY)

    def write(self, elem_offset: int, data: np.ndarray, min_bytes: int = 4 << 20) -> None:
        """data (contiguous, this file's dtype) at element `elem_offset` of the flat array."""
        buf = memoryview(np.ascontiguousarray(data)).cast("B")
        pos = self.offset + elem_offset * self.dtype.itemsize
        n = len(buf)
        parts = 1 if n < min_bytes else _COPY_THREADS
        bounds = [n * i // parts // 4096 * 4096 for i in range(parts)] + [n]

        def one(i):
            lo, hi = bounds[i], bounds[i + 1]
            while lo < hi:
                lo += os.pwrite(self.fd, buf[lo:hi], pos + lo)
        if parts == 1:
            one(0)
        else:
            list(_copy_pool().map(one, range(parts)))

    def close(self) -> None:
        if self.fd >= 0:
            os.close(self.fd)
            self.fd = -1


def _par_copy(dst: np.ndarray, src: np.ndarray, min_bytes: int = 4 << 20) -> None:
    """dst[...] = src, split over the copy threads along axis 0 when it is large."""
    n = dst.shape[0] if dst.ndim else 0
    if dst.nbytes < min_bytes or n < 2:
        dst[...] = src
        return
    parts = min(_COPY_THREADS, n)
    bounds = [n * i // parts for i in range(parts + 1)]

    def one(i):
        dst[bounds[i]:bounds[i + 1]] = src[bounds[i]:bounds[i + 1]]
    list(_copy_pool().map(one, range(parts)))


def _stream_compiled(pipeline, arrays, total, batch, out_name, out_path,
                     extras: Sequence[str] = ()) -> Tuple[int, ...]:
    """Compiled path with host I/O overlapped with the GPU.

    Per batch: the input slice goes through a pinned buffer (two, used in
    turn) as an asynchronous H2D on the program's stream; the program runs;
    its logits are copied on the device into one of two staging buffers.
    While the GPU runs batch i, the host drains batch i - 1: a copy stream
    moves its staging buffer to the host in 64 MB pinned chunks (two, used in
    turn), and each chunk is written into logits.npy by positioned writes
    from the copy threads.  The non-finite check (X:1177) runs on the device over
    each batch's logits (c3h_nonfinite) and only its flag crosses to the host.
    No whole-output device or host copy is ever built, so C5's 2.1 GB of
    logits cost one staging buffer per slot.  The pinned and device staging
    buffers stay with the pipeline, so a second call with the same batch
    shape allocates nothing.
    Further graph outputs (`extras`, e.g. the decoders' int64 ArgMax) are
    staged the same way and drained whole into <name>.npy.
    """
    from ..device import Event, PinnedArray, Stream

    cache = pipeline.__dict__.setdefault("_stream_buffers", {})

    def kept(key, make):
        if key not in cache:
            cache[key] = make()
        return cache[key]

    names = list(arrays)
    pin_in = [{n: kept(("in", n, slot, (batch,) + arrays[n].shape[1:], arrays[n].dtype.str),
                       lambda n=n: PinnedArray((batch,) + arrays[n].shape[1:], arrays[n].dtype))
               for n in names} for slot in range(2)]
    copy_stream = kept("copy_stream", Stream)
    stage: list = [None, None]
    ready = [Event(), Event()]
    chunks = [kept(("chunk", k), lambda: PinnedArray((_CHUNK_BYTES // 4,), np.float32)) for k in range(2)]
    chunk_done = [Event(), Event()]
    flags = [PinnedArray((1,), np.int32) for _ in range(2)]  # each batch's gather error flag
    nf_dev = [DeviceArray.empty((1,), np.int32) for _ in range(2)]  # each batch's non-finite flag
    nf_host = [PinnedArray((1,), np.int32) for _ in range(2)]
    progs: list = [None, None]
    x_stage: list = [{}, {}]   # per slot: extra output name -> device staging buffer
    x_host: list = [{}, {}]    # per slot: extra output name -> pinned host buffer
    x_mm: Dict[str, Any] = {}
    mm = None
    tail: Optional[Tuple[int, ...]] = None
    pending = None  # (slot, start, end) of the batch still on the device

    def drain(slot, start, end):
        copy_stream.wait_event(ready[slot])
        flag = progs[slot]._error_flag()
        _lib.check(_lib.lib().c3h_memcpy_d2h_async(flags[slot].ptr, flag.ptr, 4, copy_stream.handle), "d2h")
        _lib.check(_lib.lib().c3h_memcpy_d2h_async(nf_host[slot].ptr, nf_dev[slot].ptr, 4, copy_stream.handle), "d2h")
        src = stage[slot]
        row = math.prod(tail)
        first, last = start * row, end * row
        step = _CHUNK_BYTES // 4
        spans = [(o, min(o + step, last)) for o in range(first, last, step)]

        def issue(k):
            o0, o1 = spans[k]
            _lib.check(_lib.lib().c3h_memcpy_d2h_async(chunks[k % 2].ptr, src.ptr + (o0 - first) * 4, (o1 - o0) * 4,
                                                       copy_stream.handle), "d2h")
            chunk_done[k % 2].record(copy_stream)

        def check_flags():
            if int(flags[slot].array[0]) != 0:
                progs[slot].check_errors()  # clears the flag and raises IndexError
            if int(nf_host[slot].array[0]) != 0:
                raise ValueError("Output contains non-finite values (NaN or Inf)")

        if spans:
            issue(0)
        else:
            copy_stream.synchronize()
            check_flags()
        for k, (o0, o1) in enumerate(spans):
            if k + 1 < len(spans):
                issue(k + 1)
            chunk_done[k % 2].synchronize()  # the flag copies were queued before chunk 0
            if k == 0:
                check_flags()
            mm.write(o0, chunks[k % 2].array[: o1 - o0])
        if extras:
            for n in extras:
                src_x = x_stage[slot][n]
                _lib.check(_lib.lib().c3h_memcpy_d2h_async(x_host[slot][n].ptr, src_x.ptr,
                                                           (end - start) * src_x.nbytes // src_x.shape[0],
                                                           copy_stream.handle), "d2h")
            copy_stream.synchronize()
            for n in extras:
                x_mm[n][start:end] = x_host[slot][n].array[: end - start]

    try:
        for i, start in enumerate(range(0, total, batch)):
            end = min(start + batch, total)
            nb = end - start
            slot = i % 2
            prog = pipeline.compiled_for_batch(nb)
            pipeline.last_plan = pipeline._plan_for_batch(nb)
            feed = {}
            for n in names:
                view = pin_in[slot][n].array[:nb]
                _par_copy(view, arrays[n][start:end])
                feed[n] = (pin_in[slot][n], view.nbytes)
            prog.stage_inputs(feed)
            prog.launch()
            progs[slot] = prog
            out = prog.output_arrays[out_name]
            tail = _check_output(out, out_name, tail)
            # non-finite check of this batch's logits on the device (X:1177)
            fa = _lib.FillArgs()
            fa.out, fa.count, fa.dtype, fa.value = nf_dev[slot].ptr, 1, _lib.I32, 0.0
            _lib.launch(fa, prog.stream.handle)
            na = _lib.NonfiniteArgs()
            na.x, na.flag, na.count, na.dtype = out.ptr, nf_dev[slot].ptr, out.size, _lib.F32
            _lib.launch(na, prog.stream.handle)
            if mm is None:
                mm = _NpyWriter(out_path, np.float32, (total,) + tail)
            if stage[slot] is None:
                stage[slot] = kept(("stage", slot, (batch,) + tail), lambda: DeviceArray.empty((batch,) + tail, np.float32))
            _lib.check(_lib.lib().c3h_memcpy_d2d_async(stage[slot].ptr, out.ptr, out.nbytes, prog.stream.handle), "d2d")
            for n in extras:
                xo = prog.output_arrays[n]
                if n not in x_mm:
                    x_mm[n] = np.lib.format.open_memmap(_extra_path(out_path, n), mode="w+", dtype=xo.dtype,
                                                        shape=(total,) + xo.shape[1:])
                if n not in x_stage[slot]:
                    key = (n, slot, (batch,) + xo.shape[1:], xo.dtype.str)
                    x_stage[slot][n] = kept(("xstage",) + key, lambda: DeviceArray.empty((batch,) + xo.shape[1:], xo.dtype))
                    x_host[slot][n] = kept(("xhost",) + key, lambda: PinnedArray((batch,) + xo.shape[1:], xo.dtype))
                _lib.check(_lib.lib().c3h_memcpy_d2d_async(x_stage[slot][n].ptr, xo.ptr, xo.nbytes, prog.stream.handle),
                           "d2d")
            ready[slot].record(prog.stream)
            if pending is not None:
                drain(*pending)
            pending = (slot, start, end)
        if pending is None:
            raise RuntimeError("Inference produced no output batches")
        drain(*pending)
    except BaseException:
        # the cached buffers are idle again before the error propagates, and no
        # partial output file stays behind (the reference raises before it saves, X:1177-1186)
        copy_stream.synchronize()
        for p in progs:
            if p is not None:
                p.stream.synchronize()
        if mm is not None:
            mm.close()
            os.remove(out_path)
        for n in list(x_mm):
            del x_mm[n]
            os.remove(_extra_path(out_path, n))
        raise
    mm.close()
    shape = (total,) + tail
    for n in extras:
        x_mm[n].flush()
    x_mm.clear()
    return shape


def load_and_infer(model_path: str, input_dir: str, output_dir: str, batch_size: Optional[int] = None,
                   qualify_optimizations: bool = False, engine_kind: str = "compiled",
                   precision: Optional[str] = None, weights: Optional[Dict[str, Any]] = None,
                   graph: Optional[Graph] = None) -> Dict[str, Any]:
    """Load model + inputs, run all batches, write logits.npy + manifest.json (X:997-1265)."""
    from ..onnx_io import import_onnx

    t0 = time.perf_counter()
    init()
    tp = time.perf_counter()
    if graph is None:
        graph = import_onnx(model_path)
    tp_end = time.perf_counter()
    manifest_path = os.path.join(input_dir, "manifest.json")
    if not os.path.isfile(manifest_path):
        raise FileNotFoundError(f"Input manifest not found: {manifest_path}")
    with open(manifest_path) as f:
        manifest = json.load(f)
    arrays: Dict[str, np.ndarray] = {}
    for entry in manifest.get("tensors", []):
        name = entry["name"]
        if name in arrays:
            raise ValueError(f"Duplicate input tensor in manifest: '{name}'")
        path = os.path.join(input_dir, entry["file"])
        if not os.path.isfile(path):
            raise FileNotFoundError(f"Input file not found: {path}")
        arr = np.load(path, allow_pickle=False)
        if entry.get("dtype") is not None and np.dtype(entry["dtype"]) != arr.dtype:
            raise ValueError(f"Input '{name}' dtype mismatch: manifest={entry['dtype']}, npy={arr.dtype}")
        if entry.get("shape") is not None and list(arr.shape) != list(entry["shape"]):
            raise ValueError(f"Input '{name}' shape mismatch: manifest={entry['shape']}, npy={list(arr.shape)}")
        arrays[name] = arr
    if not arrays:
        raise ValueError("No input tensors found in manifest")
    expected = {t.name: t for t in graph.inputs}
    if set(arrays) != set(expected):
        raise ValueError("Input manifest names do not match graph inputs: "
                         f"missing={sorted(set(expected) - set(arrays))}, unexpected={sorted(set(arrays) - set(expected))}")
    dtype_map = {"FLOAT": np.float32, "FLOAT16": np.float16, "DOUBLE": np.float64, "INT32": np.int32,
                 "INT64": np.int64, "BOOL": np.bool_}
    for name, t in expected.items():
        arr = arrays[name]
        want = dtype_map.get(t.dtype.value)
        if want is not None and arr.dtype != np.dtype(want):
            raise ValueError(f"Input '{name}' dtype {arr.dtype} does not match graph dtype {np.dtype(want)}")
        if arr.ndim != len(t.shape):
            raise ValueError(f"Input '{name}' rank {arr.ndim} does not match graph rank {len(t.shape)}")
        for axis, (got, dim) in enumerate(zip(arr.shape, t.shape)):
            try:
                if got != int(dim):
                    raise ValueError(f"Input '{name}' dimension {axis} is {got}, expected {int(dim)}")
            except (TypeError, ValueError) as exc:
                if "dimension" in str(exc):
                    raise
    counts = {a.shape[0] for a in arrays.values()}
    if len(counts) != 1:
        raise ValueError(f"All graph inputs must have equal sample counts, got {sorted(counts)}")
    total = next(iter(counts))
    if total <= 0:
        raise ValueError("Input tensors must contain at least one sample")
    batch = total if batch_size is None or batch_size <= 0 else min(batch_size, total)
    precision = precision or "fp32"
    pipeline = CrossStageReferencePipeline(graph, weights if weights is not None else model_path,
                                           qualify_optimizations=qualify_optimizations, engine_kind=engine_kind,
                                           precision=precision)
    out_name = graph.outputs[0].name if graph.outputs else "logits"
    extras = [t.name for t in graph.outputs[1:]]
    os.makedirs(output_dir, exist_ok=True)
    out_path = os.path.join(output_dir, "logits.npy")
    ti = time.perf_counter()
    if engine_kind == "compiled":
        if qualify_optimizations:  # C3.3 check on the first batch (X:955-994), then the streamed run
            pipeline.run({name: DeviceArray.from_host(arr[:batch]) for name, arr in arrays.items()})
        out_shape = _stream_compiled(pipeline, arrays, total, batch, out_name, out_path, extras)
    else:
        out_shape = _run_planned_batches(pipeline, arrays, total, batch, out_name, out_path, extras)
    ti_end = time.perf_counter()
    with open(os.path.join(output_dir, "manifest.json"), "w") as f:
        json.dump({"tensors": [{"name": out_name, "file": "logits.npy", "dtype": "float32",
                                "shape": list(out_shape)}]}, f, indent=2)
    t_end = time.perf_counter()
    trace = pipeline.optimized_executor.last_execution_trace
    counts_by_kind = {k: sum(a["kind"] == k for a in trace)
                      for k in ("ALLOC", "H2D", "EVENT_WAIT", "KERNEL", "EVENT_RECORD", "FREE", "D2H")}
    from ..device import device_props

    props = device_props(0)
    evidence = {"device_name": props.name.decode(errors="replace"), "arch": props.arch.decode(errors="replace"),
                "compute_units": props.compute_units, "library": str(_lib.lib()._name),
                "batch_count": (total + batch - 1) // batch, "engine": engine_kind, "precision": precision}
    return {
        "model_path": model_path, "input_dir": input_dir, "output_dir": output_dir, "batch_size": batch,
        "backend": "libc3hip", "backend_evidence": evidence, "engine": engine_kind, "total_samples": total, "output_shape": list(out_shape),
        "extra_outputs": {n: os.path.basename(_extra_path(out_path, n)) for n in extras},
        "parse_time_s": tp_end - tp, "infer_time_s": ti_end - ti, "total_time_s": t_end - t0,
        "cross_stage_reference": True, "optimized_graph_nodes": len(pipeline.graph.nodes),
        "fusion_stats": pipeline.fusion_result["Fusion"]["stats"],
        "qualification_max_abs_diff": pipeline.qualification_max_abs_diff,
        "plan_summary": pipeline.last_plan.summary() if pipeline.last_plan else None,
        "plan_runtime": {"timeline_actions_consumed": len(trace), "action_counts": counts_by_kind,
                         "resources": pipeline.optimized_executor.runtime_resource_stats()},
    }
