"""Tensor lifetime analysis (counterpart of c34/lifetime.py).

first_use / last_use are kernel-schedule indices; sizes resolve symbolic batch
dims ("N", "batch", "b", "unk__*", -1) to the planned batch size
(c34/lifetime.py:36-174).
"""

from __future__ import annotations

from typing import Dict, List, Optional

from ..c3common.ir.graph import Graph
from ..c32.kernel_spec import KernelSpecRef
from .execution_plan import LifetimeInterval

DTYPE_SIZE_BYTES = {
    "FLOAT": 4, "FLOAT16": 2, "BFLOAT16": 2, "DOUBLE": 8, "INT8": 1, "UINT8": 1, "BOOL": 1,
    "INT16": 2, "UINT16": 2, "INT32": 4, "UINT32": 4, "INT64": 8, "UINT64": 8,
}


def resolve_dim(d, batch_size: int) -> Optional[int]:
    """Concrete value of one dimension, or None when it is unknown."""
    if d is None:
        return None
    try:
        v = int(d)
    except (TypeError, ValueError):
        if isinstance(d, str) and (d.lower() in ("n", "batch", "b") or d.startswith("unk__")):
            return batch_size
        return None
    if v == -1:
        return batch_size
    return v if v >= 0 else None


def _compute_size_with_batch(shape: list, batch_size: int = 1, elem_bytes: int = 4) -> int:
    total = elem_bytes
    for d in shape:
        v = resolve_dim(d, batch_size)
        if v is None:
            return 0
        total *= v
    return total


def _tensor_size_bytes(graph: Graph, name: str, batch_size: int = 1) -> int:
    t = graph.tensors.get(name)
    if t is None:
        return 0
    elem = DTYPE_SIZE_BYTES.get(t.dtype.value, 4)
    if (t.is_constant or t.is_initializer) and not t.shape:
        return elem  # rank-0 constant / initializer: one element (the reference sized these 0)
    return _compute_size_with_batch(t.shape, batch_size, elem) if t.shape else 0


def _find_node_id_for_tensor(graph: Graph, name: str) -> Optional[str]:
    p = graph.tensor_producer.get(name)
    return p if p and p not in ("INPUT", "INITIALIZER", "CONSTANT") else None


def compute_lifetimes(graph: Graph, kernel_schedule: List[KernelSpecRef],
                      batch_size: int = 1) -> Dict[str, LifetimeInterval]:
    inputs = {t.name for t in graph.inputs}
    outputs = {t.name for t in graph.outputs}
    inits = set(graph.initializers)
    first: Dict[str, int] = {}
    last: Dict[str, int] = {}
    producers: Dict[str, List[str]] = {}
    consumers: Dict[str, List[int]] = {}
    for step, k in enumerate(kernel_schedule):
        for name in k.inputs:
            if name:
                first.setdefault(name, step)
                last[name] = step
                consumers.setdefault(name, []).append(step)
        for name in k.outputs:
            if name:
                first.setdefault(name, step)
                last[name] = step
                plist = producers.setdefault(name, [])
                nid = _find_node_id_for_tensor(graph, name)
                if nid and nid not in plist:
                    plist.append(nid)
    lifetimes: Dict[str, LifetimeInterval] = {}
    for name, f in first.items():
        t = graph.tensors.get(name)
        lifetimes[name] = LifetimeInterval(
            tensor_name=name, first_use=f, last_use=last[name],
            size_bytes=_tensor_size_bytes(graph, name, batch_size),
            is_weight=name in inits or bool(t is not None and t.is_constant),
            is_output=name in outputs, is_input=name in inputs and name not in inits,
            producers=producers.get(name, []), consumers=[str(i) for i in consumers.get(name, [])])
    return lifetimes


def find_overlap_groups(lifetimes: Dict[str, LifetimeInterval]) -> List[List[LifetimeInterval]]:
    """Greedy interval grouping of tensors that could share one slot."""
    groups: List[List[LifetimeInterval]] = []
    for li in sorted(lifetimes.values(), key=lambda x: (x.first_use, x.last_use)):
        if li.is_weight or li.is_input:
            groups.append([li])
            continue
        for g in groups:
            if any(x.is_weight or x.is_input for x in g):
                continue
            if max(x.last_use for x in g) < li.first_use:
                g.append(li)
                break
        else:
            groups.append([li])
    return groups
