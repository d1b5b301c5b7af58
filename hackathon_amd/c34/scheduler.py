"""Execution-plan builder (counterpart of c34/scheduler.py).

Produces the same plan the reference planner produces for a graph
(c34/scheduler.py:93-1135): a flat kernel schedule of every C3.2 step,
lifetimes, weight/input slots and H2D transfers on copy stream 0,
lifetime-reusing intermediate slots from a best-fit pool, compute streams
assigned round-robin by DAG depth (at most 4), cross-stream / arena-reuse /
output-ready events, D2H readback of graph outputs and one interleaved
timeline.  Two differences: the producer/consumer searches use index maps
instead of nested scans, and the strategy carries this build's
PrecisionPolicy so 16-bit / int8 profiles reach KernelStep.precision_profile
(the reference hard-codes FULL_FP32, c34/scheduler.py:70).
"""

from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Set, Tuple

from ..c3common.ir.graph import Graph, ONNSType
from ..c32.kernel_spec import KernelSpecRef
from ..c32.strategy import ExecutionMode, PrecisionPolicy, Strategy
from .execution_plan import (Allocation, EventDep, ExecutionPlan, KernelStep, LifetimeInterval,
                             TimelineStep, Transfer)
from .lifetime import compute_lifetimes
from .memory_pool import DeviceMemoryPool, FitPolicy

COPY_STREAM = 0
FIRST_COMPUTE_STREAM = 1
MAX_COMPUTE_STREAMS = 4


class ExecutionScheduler:
    def __init__(self, graph: Graph, batch_size: int = 1, enable_prefetch: bool = True,
                 enable_multi_stream: bool = True, pool_policy: str = FitPolicy.BEST_FIT,
                 precision_policy: Optional[PrecisionPolicy] = None) -> None:
        self.graph = graph
        self.batch_size = batch_size
        self.enable_prefetch = enable_prefetch
        self.enable_multi_stream = enable_multi_stream
        self.pool_policy = pool_policy
        self._strategy = Strategy(mode=ExecutionMode.FULL_FP32, policy=precision_policy)
        self._pool = DeviceMemoryPool(policy=pool_policy)
        self._allocations: List[Allocation] = []
        self._transfers: List[Transfer] = []
        self._kernel_steps: List[KernelStep] = []
        self._events: List[EventDep] = []
        self._event_ids: Set[str] = set()
        self._weight_slots: Dict[str, str] = {}
        self._alloc_map: Dict[str, str] = {}
        self._kernel_schedule: List[KernelSpecRef] = []
        self._kernel_node_map: Dict[int, str] = {}
        self._node_decompositions: Dict[str, List[str]] = {}
        self._node_precisions: Dict[str, Dict[str, Optional[str]]] = {}
        self._timeline: List[TimelineStep] = []

    def build(self) -> ExecutionPlan:
        self._build_kernel_schedule()
        lifetimes = compute_lifetimes(self.graph, self._kernel_schedule, self.batch_size)
        self._allocate_weights(lifetimes)
        self._allocate_inputs(lifetimes)
        self._allocate_intermediates(lifetimes)
        self._schedule_kernels()
        self._schedule_output_readback(lifetimes)
        self._add_reuse_dependencies(lifetimes)
        self._add_output_dependencies()
        self._build_timeline(lifetimes)
        return ExecutionPlan(
            model_name=self.graph.name, batch_size=self.batch_size, allocations=self._allocations,
            transfers=self._transfers, kernel_steps=self._kernel_steps, events=self._events,
            timeline=self._timeline, lifetimes=lifetimes, pool_stats=self._pool.stats(),
            weight_slots=self._weight_slots,
            num_compute_streams=len({FIRST_COMPUTE_STREAM} | {k.stream_id for k in self._kernel_steps}),
            copy_stream_id=COPY_STREAM)

    # -- step 1: flat kernel schedule -----------------------------------------------
    def _build_kernel_schedule(self) -> None:
        if not self.graph.node_order:
            self.graph.topological_sort()
        for nid in self.graph.node_order:
            node = self.graph.nodes.get(nid)
            if node is None:
                continue
            precision = self._strategy.select_precision(node, self.graph)
            kernels = self._strategy.decompose(node, self.graph, precision)
            self._node_decompositions[nid] = [k.kernel_name for k in kernels]
            self._node_precisions[nid] = precision.as_dict()
            for k in kernels:
                self._register_intermediate_tensors(node, k)
                k.tuning_params = self._strategy.tune_kernel(k, precision)
                k.precision_profile = precision
                k.operator_params.setdefault("_batch_size", self.batch_size)
                self._kernel_node_map[len(self._kernel_schedule)] = nid
                self._kernel_schedule.append(k)

    def _register_intermediate_tensors(self, node, k: KernelSpecRef) -> None:
        dtype = next((self.graph.tensors[o].dtype for o in node.outputs
                      if o in self.graph.tensors and self.graph.tensors[o].dtype != ONNSType.UNDEFINED),
                     ONNSType.FLOAT)
        shape = self._infer_output_shape(node, k)
        for o in k.outputs:
            if o and o not in node.outputs and o not in self.graph.tensors:
                self.graph.register_tensor(o, dtype=dtype, shape=shape)

    def _resolve(self, shape) -> List[int]:
        out = []
        for d in shape:
            if d is None:
                return []
            try:
                out.append(int(d))
            except (TypeError, ValueError):
                if isinstance(d, str) and (d.lower() in ("n", "batch", "b") or d.startswith("unk__")):
                    out.append(self.batch_size)
                else:
                    return []
        return out

    def _shape_of(self, name: str) -> List[int]:
        t = self.graph.tensors.get(name)
        return self._resolve(t.shape) if t is not None and t.shape else []

    def _infer_output_shape(self, node, k: KernelSpecRef) -> List[int]:
        """Intermediate shape from the parent node (c34/scheduler.py:225-404)."""
        name = k.kernel_name
        if {o for o in k.outputs if o} & set(node.outputs):
            for o in node.outputs:
                s = self._shape_of(o)
                if s:
                    return s
        in_shapes = [s for s in (self._shape_of(i) for i in k.inputs) if s]
        if name.startswith("matmul") and len(in_shapes) >= 2:
            a, b = in_shapes[0], in_shapes[1]
            if k.operator_params.get("lowering_kind", "") == "conv_contract":
                return [a[-2] if len(a) >= 2 else 1, b[0] if b else 1]
            m = a[-2] if len(a) >= 2 else 1
            n = b[-2] if node.attributes.get("transB", 0) else b[-1]
            return a[:-2] + [m, n] if len(a) >= 3 else [m, n]
        if name.startswith("im2col") and in_shapes:
            s = in_shapes[0]
            p = k.operator_params
            ks = p.get("kernel_shape", [3, 3])
            kh, kw = int(ks[0]), int(ks[-1]) if len(ks) > 1 else int(ks[0])
            if len(s) == 4:
                n, c, h, w = s
                st, dl = p.get("strides", [1, 1]), p.get("dilations", [1, 1])
                pt, pl, pb, pr = [int(v) for v in p.get("pads", [0, 0, 0, 0])]
                ho = (h + pt + pb - int(dl[0]) * (kh - 1) - 1) // int(st[0]) + 1
                wo = (w + pl + pr - int(dl[-1]) * (kw - 1) - 1) // int(st[-1]) + 1
                if ho > 0 and wo > 0:
                    return [n * ho * wo, c * kh * kw]
            return [math.prod(s) * kh * kw]
        if name.startswith("winograd"):
            # The convolution's output shape is the node's (the reference used
            # the input's, which undersizes channel-expanding convolutions).
            for o in node.outputs:
                s = self._shape_of(o)
                if s:
                    return s
        if name.startswith(("add", "mul", "div", "sub", "relu", "erf", "sqrt", "exp", "reciprocal",
                            "reduce_", "gather", "reshape", "transpose", "split", "constant")):
            if in_shapes:
                return in_shapes[0]
        if name == "flatten" and in_shapes and len(in_shapes[0]) >= 2:
            return [in_shapes[0][0], math.prod(in_shapes[0][1:])]
        for o in node.outputs:
            s = self._shape_of(o)
            if s:
                return s
        return in_shapes[0] if in_shapes else []

    # -- step 3: weights and inputs ----------------------------------------------------
    def _allocation(self, alloc_id: str, tensor_name: str, slot_id: int, size_bytes: int,
                    is_weight: bool = False, is_output: bool = False) -> Allocation:
        offset, capacity = self._pool.describe(slot_id)
        return Allocation(alloc_id=alloc_id, tensor_name=tensor_name, slot_id=slot_id, size_bytes=size_bytes,
                          is_weight=is_weight, is_output=is_output, offset_bytes=offset, capacity_bytes=capacity)

    def _add_event(self, event_id: str, src: int, dst: int, description: str) -> None:
        if event_id not in self._event_ids:
            self._event_ids.add(event_id)
            self._events.append(EventDep(event_id, src, dst, description))

    def _allocate_weights(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        for name in sorted(lifetimes):
            li = lifetimes[name]
            if not li.is_weight or li.size_bytes <= 0:
                continue
            slot = self._pool.alloc(li.size_bytes)
            aid = f"alloc_w_{name}"
            self._allocations.append(self._allocation(aid, name, slot, li.size_bytes,
                                                      is_weight=name in self.graph.initializers))
            self._weight_slots[name] = aid
            self._alloc_map[name] = aid
            eid = f"evt_wready_{name}"
            self._transfers.append(Transfer("H2D", name, aid, li.size_bytes, COPY_STREAM, eid))
            self._add_event(eid, COPY_STREAM, FIRST_COMPUTE_STREAM, f"Weight ready: {name}")

    def _allocate_inputs(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        for name in sorted(lifetimes):
            li = lifetimes[name]
            if not li.is_input or li.size_bytes <= 0:
                continue
            slot = self._pool.alloc(li.size_bytes)
            aid = f"alloc_in_{name}"
            self._allocations.append(self._allocation(aid, name, slot, li.size_bytes))
            self._alloc_map[name] = aid
            eid = f"evt_input_ready_{name}"
            self._transfers.append(Transfer("H2D", name, aid, li.size_bytes, COPY_STREAM, eid))
            self._add_event(eid, COPY_STREAM, FIRST_COMPUTE_STREAM, f"Input ready: {name}")

    # -- step 4: intermediates with reuse ------------------------------------------------
    def _allocate_intermediates(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        inter = sorted((li for li in lifetimes.values()
                        if not li.is_weight and not li.is_input and li.size_bytes > 0),
                       key=lambda li: (li.first_use, li.last_use))
        alloc_before: Dict[int, List[LifetimeInterval]] = {}
        free_after: Dict[int, List[str]] = {}
        for li in inter:
            alloc_before.setdefault(li.first_use, []).append(li)
            if not li.is_output:
                free_after.setdefault(li.last_use, []).append(li.tensor_name)
        slot_of: Dict[str, int] = {}
        steps = len(self._kernel_schedule)
        for step in range(steps + 1):
            if step < steps:
                for li in alloc_before.get(step, []):
                    if li.tensor_name in self._alloc_map:
                        continue
                    slot = self._pool.alloc(li.size_bytes)
                    aid = f"alloc_{li.tensor_name}"
                    if len(aid) > 64:
                        aid = f"alloc_inter_{slot}_{len(self._allocations)}"
                    self._allocations.append(self._allocation(aid, li.tensor_name, slot, li.size_bytes,
                                                              is_output=li.is_output))
                    self._alloc_map[li.tensor_name] = aid
                    slot_of[li.tensor_name] = slot
            for name in free_after.get(step, []):
                if name in slot_of and name not in self._weight_slots:
                    self._pool.free(slot_of.pop(name))

    # -- step 5: kernel steps, streams, events -----------------------------------------------
    def _producer_index(self) -> Dict[str, int]:
        producer: Dict[str, int] = {}
        for i, k in enumerate(self._kernel_schedule):
            for o in k.outputs:
                if o and o not in producer:
                    producer[o] = i
        return producer

    def _assign_streams(self) -> Dict[int, int]:
        n = len(self._kernel_schedule)
        if n <= 1:
            return {0: FIRST_COMPUTE_STREAM}
        producer = self._producer_index()
        depth: Dict[int, int] = {}
        for j, k in enumerate(self._kernel_schedule):
            preds = {producer[i] for i in k.inputs if i in producer and producer[i] < j}
            depth[j] = 1 + max((depth[p] for p in preds), default=-1)
        counters: Dict[int, int] = {}
        out: Dict[int, int] = {}
        for j in range(n):
            c = counters.get(depth[j], 0)
            out[j] = FIRST_COMPUTE_STREAM + c % MAX_COMPUTE_STREAMS
            counters[depth[j]] = c + 1
        return out

    def _schedule_kernels(self) -> None:
        streams = self._assign_streams() if self.enable_multi_stream else {}
        weight_events = {t.tensor_name: t.event_id for t in self._transfers
                         if t.kind == "H2D" and t.tensor_name in self._weight_slots and t.event_id}
        input_events = {t.tensor_name: t.event_id for t in self._transfers
                        if t.kind == "H2D" and t.tensor_name not in self._weight_slots and t.event_id}
        producer = self._producer_index()
        for j, k in enumerate(self._kernel_schedule):
            nid = self._kernel_node_map.get(j, "unknown")
            sid = streams.get(j, FIRST_COMPUTE_STREAM)
            deps = [weight_events[i] for i in k.inputs if i in weight_events]
            deps += [input_events[i] for i in k.inputs if i in input_events]
            if self.enable_multi_stream:
                for i in k.inputs:
                    p = producer.get(i)
                    if not i or p is None or p >= j:
                        continue
                    ps = streams.get(p, FIRST_COMPUTE_STREAM)
                    if ps == sid:
                        continue
                    eid = f"evt_xs_{p}_{j}_{i}"
                    self._add_event(eid, ps, sid, f"Cross-stream: kernel {p} (stream {ps}) -> kernel {j} "
                                                  f"(stream {sid}) via {i}")
                    if eid not in self._kernel_steps[p].signals:
                        self._kernel_steps[p].signals.append(eid)
                    deps.append(eid)
            tp = k.tuning_params
            self._kernel_steps.append(KernelStep(
                step_index=j, kernel_name=k.kernel_name, node_id=nid,
                logical_inputs=[i for i in k.inputs if i], logical_outputs=[o for o in k.outputs if o],
                inputs={i: self._alloc_map[i] for i in k.inputs if i and i in self._alloc_map},
                outputs={o: self._alloc_map[o] for o in k.outputs if o and o in self._alloc_map},
                stream_id=sid, depends_on=deps, signals=[],
                tuning_params=None if tp is None else {"block_x": tp.block_x, "grid_x": tp.grid_x,
                                                       "smem_bytes": tp.smem_bytes},
                operator_params=dict(k.operator_params), precision_profile=dict(self._node_precisions[nid]),
                lowered_kernels=list(self._node_decompositions.get(nid, []))))

    def _schedule_output_readback(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        for name in sorted({t.name for t in self.graph.outputs}):
            li = lifetimes.get(name)
            size = li.size_bytes if li else 0
            if name not in self._alloc_map:
                if size <= 0:
                    continue
                slot = self._pool.alloc(size)
                aid = f"alloc_out_{name}"
                self._allocations.append(self._allocation(aid, name, slot, size, is_output=True))
                self._alloc_map[name] = aid
            self._transfers.append(Transfer("D2H", name, self._alloc_map[name], size, COPY_STREAM))

    @staticmethod
    def _ranges_overlap(a: Allocation, b: Allocation) -> bool:
        return (a.offset_bytes < b.offset_bytes + (b.capacity_bytes or b.size_bytes)
                and b.offset_bytes < a.offset_bytes + (a.capacity_bytes or a.size_bytes))

    def _add_reuse_dependencies(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        """Happens-before edges between cross-stream users of a reused byte range."""
        for cur in self._allocations:
            cl = lifetimes.get(cur.tensor_name)
            if cl is None or cl.is_weight:
                continue
            best: Optional[Tuple[int, Allocation]] = None
            for prev in self._allocations:
                pl = lifetimes.get(prev.tensor_name)
                if prev.alloc_id == cur.alloc_id or pl is None or not self._ranges_overlap(prev, cur):
                    continue
                if pl.last_use < cl.first_use and (best is None or pl.last_use > best[0]):
                    best = (pl.last_use, prev)
            if best is None:
                continue
            src_i, prev = best
            dst_i = cl.first_use
            if not (0 <= src_i < len(self._kernel_steps) and 0 <= dst_i < len(self._kernel_steps)):
                continue
            src, dst = self._kernel_steps[src_i], self._kernel_steps[dst_i]
            if src.stream_id == dst.stream_id:
                continue
            eid = f"evt_reuse_{src_i}_{dst_i}_{prev.slot_id}_{cur.slot_id}"
            self._add_event(eid, src.stream_id, dst.stream_id,
                            f"Arena reuse: {prev.tensor_name} -> {cur.tensor_name}")
            if eid not in src.signals:
                src.signals.append(eid)
            if eid not in dst.depends_on:
                dst.depends_on.append(eid)

    def _add_output_dependencies(self) -> None:
        last_producer: Dict[str, int] = {}
        for i, k in enumerate(self._kernel_steps):
            for o in k.logical_outputs:
                last_producer[o] = i
        for t in self._transfers:
            if t.kind != "D2H" or t.tensor_name not in last_producer:
                continue
            prod = self._kernel_steps[last_producer[t.tensor_name]]
            eid = f"evt_output_ready_{t.tensor_name}"
            self._add_event(eid, prod.stream_id, t.stream_id, f"Output ready: {t.tensor_name}")
            if eid not in prod.signals:
                prod.signals.append(eid)
            if eid not in t.depends_on:
                t.depends_on.append(eid)

    # -- step 7: unified timeline ---------------------------------------------------------------
    def _build_timeline(self, lifetimes: Dict[str, LifetimeInterval]) -> None:
        actions: List[TimelineStep] = []

        def emit(kind: str, **kw: Any) -> None:
            actions.append(TimelineStep(step_index=len(actions), kind=kind, **kw))

        alloc_by_tensor = {a.tensor_name: a for a in self._allocations}
        h2d_at: Dict[int, List[int]] = {}
        d2h: List[int] = []
        for idx, t in enumerate(self._transfers):
            if t.kind == "D2H":
                d2h.append(idx)
                continue
            li = lifetimes.get(t.tensor_name)
            first = li.first_use if li is not None else 0
            at = first - 1 if self.enable_prefetch and t.tensor_name in self._weight_slots and first > 0 else 0
            h2d_at.setdefault(at, []).append(idx)
        first_at: Dict[int, List[str]] = {}
        last_at: Dict[int, List[str]] = {}
        for name in sorted(lifetimes):
            li = lifetimes[name]
            first_at.setdefault(li.first_use, []).append(name)
            last_at.setdefault(li.last_use, []).append(name)
        allocated: Set[str] = set()
        freed: Set[str] = set()
        zero = LifetimeInterval("", 0, 0, 0)
        for ki, k in enumerate(self._kernel_steps):
            staged = sorted(h2d_at.get(ki, []), key=lambda i: (
                lifetimes.get(self._transfers[i].tensor_name, zero).first_use, self._transfers[i].tensor_name))
            for ti in staged:
                t = self._transfers[ti]
                a = alloc_by_tensor.get(t.tensor_name)
                if a is not None and a.alloc_id not in allocated:
                    emit("ALLOC", alloc_id=a.alloc_id, tensor_name=a.tensor_name)
                    allocated.add(a.alloc_id)
                emit("H2D", stream_id=t.stream_id, ref_index=ti, tensor_name=t.tensor_name)
                if t.event_id is not None:
                    emit("EVENT_RECORD", stream_id=t.stream_id, event_id=t.event_id, tensor_name=t.tensor_name)
            for name in first_at.get(ki, []):
                a = alloc_by_tensor.get(name)
                if a is not None and a.alloc_id not in allocated:
                    emit("ALLOC", alloc_id=a.alloc_id, tensor_name=name)
                    allocated.add(a.alloc_id)
            for eid in dict.fromkeys(k.depends_on):
                emit("EVENT_WAIT", stream_id=k.stream_id, event_id=eid)
            emit("KERNEL", stream_id=k.stream_id, ref_index=ki)
            for eid in dict.fromkeys(k.signals):
                emit("EVENT_RECORD", stream_id=k.stream_id, event_id=eid)
            for name in last_at.get(ki, []):
                li = lifetimes[name]
                if li.is_weight or li.is_input or li.is_output:
                    continue
                a = alloc_by_tensor.get(name)
                if a is None or a.alloc_id in freed:
                    continue
                emit("FREE", alloc_id=a.alloc_id, tensor_name=name)
                freed.add(a.alloc_id)
        for ti in d2h:
            t = self._transfers[ti]
            for eid in dict.fromkeys(t.depends_on):
                emit("EVENT_WAIT", stream_id=t.stream_id, event_id=eid, tensor_name=t.tensor_name)
            emit("D2H", stream_id=t.stream_id, ref_index=ti, tensor_name=t.tensor_name)
        self._timeline = actions
