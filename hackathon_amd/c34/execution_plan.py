"""Execution-plan data structures (counterpart of c34/execution_plan.py).

Field names and meanings are the reference's (c34/execution_plan.py:17-175):
the executor consumes plans only through these fields.  `validate()` checks
the same invariants with the same issue texts (:191-414); the live-range
overlap check is a sweep over byte-sorted allocations instead of the
reference's all-pairs loop, so validating a large plan stays cheap.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional


@dataclass
class Allocation:
    alloc_id: str
    tensor_name: str
    slot_id: int
    size_bytes: int
    alignment: int = 64
    is_weight: bool = False
    is_output: bool = False
    offset_bytes: int = 0
    capacity_bytes: int = 0


@dataclass
class Transfer:
    kind: str
    tensor_name: str
    alloc_id: str
    size_bytes: int
    stream_id: int
    event_id: Optional[str] = None
    depends_on: List[str] = field(default_factory=list)


@dataclass
class KernelStep:
    step_index: int
    kernel_name: str
    node_id: str
    logical_inputs: List[str] = field(default_factory=list)
    logical_outputs: List[str] = field(default_factory=list)
    inputs: Dict[str, str] = field(default_factory=dict)
    outputs: Dict[str, str] = field(default_factory=dict)
    stream_id: int = 1
    depends_on: List[str] = field(default_factory=list)
    signals: List[str] = field(default_factory=list)
    tuning_params: Optional[Dict[str, int]] = None
    operator_params: Dict[str, Any] = field(default_factory=dict)
    precision_profile: Optional[Dict[str, Optional[str]]] = None
    lowered_kernels: List[str] = field(default_factory=list)


@dataclass
class EventDep:
    event_id: str
    src_stream: int
    dst_stream: int
    description: str = ""


@dataclass
class TimelineStep:
    step_index: int
    kind: str
    stream_id: int = 0
    ref_index: Optional[int] = None
    alloc_id: Optional[str] = None
    event_id: Optional[str] = None
    tensor_name: Optional[str] = None


@dataclass
class LifetimeInterval:
    tensor_name: str
    first_use: int
    last_use: int
    size_bytes: int
    is_weight: bool = False
    is_output: bool = False
    is_input: bool = False
    producers: List[str] = field(default_factory=list)
    consumers: List[str] = field(default_factory=list)


@dataclass
class PoolStats:
    requested_bytes: int = 0
    reserved_bytes: int = 0
    active_bytes: int = 0
    peak_reserved_bytes: int = 0
    internal_fragmentation: int = 0
    reuse_hits: int = 0
    total_allocs: int = 0
    total_frees: int = 0
    free_list_blocks: int = 0


TIMELINE_KINDS = {"ALLOC", "FREE", "H2D", "D2H", "EVENT_WAIT", "EVENT_RECORD", "KERNEL"}


@dataclass
class ExecutionPlan:
    model_name: str = ""
    batch_size: int = 1
    allocations: List[Allocation] = field(default_factory=list)
    transfers: List[Transfer] = field(default_factory=list)
    kernel_steps: List[KernelStep] = field(default_factory=list)
    events: List[EventDep] = field(default_factory=list)
    timeline: List[TimelineStep] = field(default_factory=list)
    lifetimes: Dict[str, LifetimeInterval] = field(default_factory=dict)
    pool_stats: PoolStats = field(default_factory=PoolStats)
    weight_slots: Dict[str, str] = field(default_factory=dict)
    num_compute_streams: int = 1
    copy_stream_id: int = 0

    @property
    def peak_memory_bytes(self) -> int:
        return self.pool_stats.peak_reserved_bytes

    def summary(self) -> Dict[str, Any]:
        mb = 1024 * 1024
        return {
            "model": self.model_name, "batch_size": self.batch_size,
            "total_kernels": len(self.kernel_steps), "total_allocations": len(self.allocations),
            "total_transfers": len(self.transfers), "total_events": len(self.events),
            "timeline_steps": len(self.timeline), "weight_slots": len(self.weight_slots),
            "peak_reserved_mb": self.pool_stats.peak_reserved_bytes / mb,
            "reuse_hits": self.pool_stats.reuse_hits,
            "internal_fragmentation_mb": self.pool_stats.internal_fragmentation / mb,
            "num_compute_streams": self.num_compute_streams,
            "free_list_blocks": self.pool_stats.free_list_blocks,
        }

    def validate(self) -> List[str]:
        """Structural checks; returns the list of issues (empty = valid)."""
        issues: List[str] = []
        alloc_ids = {a.alloc_id for a in self.allocations}
        event_ids = {e.event_id for e in self.events}
        producer_step: Dict[str, int] = {}
        for k in self.kernel_steps:
            for t in k.logical_outputs:
                if t:
                    producer_step[t] = k.step_index

        for k in self.kernel_steps:
            tag = f"Kernel step {k.step_index} '{k.kernel_name}'"
            for t in k.logical_inputs:
                if t and t not in k.inputs:
                    issues.append(f"{tag} is missing input binding for '{t}'")
                p = producer_step.get(t)
                if p is not None and p >= k.step_index:
                    issues.append(f"{tag} consumes '{t}' before producer step {p}")
            for t, aid in k.inputs.items():
                if aid not in alloc_ids:
                    issues.append(f"{tag} input '{t}' references unknown alloc_id '{aid}'")
            for t in k.logical_outputs:
                if t and t not in k.outputs:
                    issues.append(f"{tag} is missing output binding for '{t}'")
            for t, aid in k.outputs.items():
                if aid not in alloc_ids:
                    issues.append(f"{tag} output '{t}' references unknown alloc_id '{aid}'")
            for e in k.depends_on:
                if e not in event_ids:
                    issues.append(f"Kernel step {k.step_index} depends on unknown event '{e}'")
            for e in k.signals:
                if e not in event_ids:
                    issues.append(f"Kernel step {k.step_index} signals unknown event '{e}'")
            if k.tuning_params is None:
                issues.append(f"{tag} has no tuning parameters")
            else:
                bx = int(k.tuning_params.get("block_x", 0))
                gx = int(k.tuning_params.get("grid_x", 0))
                sm = int(k.tuning_params.get("smem_bytes", -2))
                if bx <= 0:
                    issues.append(f"Kernel step {k.step_index} has invalid block_x={bx}")
                if gx <= 0:
                    issues.append(f"Kernel step {k.step_index} has invalid grid_x={gx}")
                if sm < -1:
                    issues.append(f"Kernel step {k.step_index} has invalid smem_bytes={sm}")
            if k.precision_profile is None:
                issues.append(f"{tag} has no precision profile")

        for t in self.transfers:
            if t.alloc_id not in alloc_ids:
                issues.append(f"Transfer '{t.kind}' for '{t.tensor_name}' references unknown alloc_id '{t.alloc_id}'")
        for name, aid in self.weight_slots.items():
            if aid not in alloc_ids:
                issues.append(f"Weight slot '{name}' references unknown alloc_id '{aid}'")

        signalled = {t.event_id for t in self.transfers if t.event_id is not None}
        signalled |= {e for k in self.kernel_steps for e in k.signals}
        waited = {e for k in self.kernel_steps for e in k.depends_on}
        waited |= {e for t in self.transfers for e in t.depends_on}
        for e in sorted(waited - signalled):
            issues.append(f"Event '{e}' is waited on but never signalled")

        issues.extend(self._overlap_issues())
        issues.extend(self._timeline_issues(alloc_ids, event_ids))
        return issues

    def _overlap_issues(self) -> List[str]:
        """Byte ranges may be shared only by tensors with disjoint lifetimes."""
        spans = []
        for idx, a in enumerate(self.allocations):
            life = self.lifetimes.get(a.tensor_name)
            if life is None:
                continue
            cap = a.capacity_bytes or a.size_bytes
            spans.append((a.offset_bytes, a.offset_bytes + cap, idx, life))
        spans.sort(key=lambda s: (s[0], s[2]))
        issues: List[str] = []
        active: List[tuple] = []
        for start, end, idx, life in spans:
            active = [s for s in active if s[1] > start]
            for _, _, oidx, olife in active:
                if not (olife.last_use < life.first_use or life.last_use < olife.first_use):
                    first, second = sorted((oidx, idx))
                    issues.append("Physical allocation overlap for live tensors "
                                  f"'{self.allocations[first].tensor_name}' and "
                                  f"'{self.allocations[second].tensor_name}'")
            active.append((start, end, idx, life))
        return issues

    def _timeline_issues(self, alloc_ids, event_ids) -> List[str]:
        issues: List[str] = []
        transfer_refs: List[int] = []
        kernel_refs: List[int] = []
        recorded: Dict[str, int] = {}
        for pos, act in enumerate(self.timeline):
            if act.step_index != pos:
                issues.append(f"Timeline index {act.step_index} is not contiguous at position {pos}")
            if act.kind not in TIMELINE_KINDS:
                issues.append(f"Unknown timeline action '{act.kind}'")
                continue
            if act.kind in ("ALLOC", "FREE"):
                if act.alloc_id not in alloc_ids:
                    issues.append(f"Timeline {act.kind} references unknown allocation '{act.alloc_id}'")
            elif act.kind in ("H2D", "D2H"):
                if act.ref_index is None or not 0 <= act.ref_index < len(self.transfers):
                    issues.append(f"Timeline {act.kind} has invalid transfer index {act.ref_index}")
                else:
                    transfer_refs.append(act.ref_index)
                    if self.transfers[act.ref_index].kind != act.kind:
                        issues.append(f"Timeline {act.kind} references "
                                      f"{self.transfers[act.ref_index].kind} transfer {act.ref_index}")
            elif act.kind == "KERNEL":
                if act.ref_index is None or not 0 <= act.ref_index < len(self.kernel_steps):
                    issues.append(f"Timeline KERNEL has invalid kernel index {act.ref_index}")
                else:
                    kernel_refs.append(act.ref_index)
            else:
                if act.event_id not in event_ids:
                    issues.append(f"Timeline {act.kind} references unknown event '{act.event_id}'")
                elif act.kind == "EVENT_RECORD":
                    recorded.setdefault(act.event_id, pos)
                elif act.event_id not in recorded:
                    issues.append(f"Timeline waits on event '{act.event_id}' before its record operation is enqueued")
        if self.timeline:
            if sorted(transfer_refs) != list(range(len(self.transfers))):
                issues.append("Timeline does not execute every transfer exactly once")
            if sorted(kernel_refs) != list(range(len(self.kernel_steps))):
                issues.append("Timeline does not execute every kernel exactly once")
        return issues
