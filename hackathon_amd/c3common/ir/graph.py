"""Graph IR shared by the planning stages (counterpart of c3common/ir/graph.py).

Field names, producer/consumer bookkeeping and method semantics follow the
reference IR (c3common/ir/graph.py:13-485) because every later stage - the
fusion passes, the decomposition table and the C3.4 plan - addresses tensors
and nodes through exactly this structure.  The implementation is this
package's own: a heap-based Kahn sort (same order as the reference's
"sorted ready list, smallest id first", :194-233) and set-based maps.
"""

from __future__ import annotations

import heapq
import math
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, List, Optional

SPECIAL_PRODUCERS = ("INPUT", "INITIALIZER", "CONSTANT")


class ONNSType(str, Enum):
    """ONNX TensorProto element types by name (c3common/ir/graph.py:13-52)."""

    UNDEFINED = "UNDEFINED"
    FLOAT = "FLOAT"
    UINT8 = "UINT8"
    INT8 = "INT8"
    UINT16 = "UINT16"
    INT16 = "INT16"
    INT32 = "INT32"
    INT64 = "INT64"
    STRING = "STRING"
    BOOL = "BOOL"
    FLOAT16 = "FLOAT16"
    DOUBLE = "DOUBLE"
    UINT32 = "UINT32"
    UINT64 = "UINT64"
    BFLOAT16 = "BFLOAT16"

    @classmethod
    def from_onnx(cls, data_type: int) -> "ONNSType":
        return _ONNX_CODES.get(int(data_type), cls.UNDEFINED)

    def to_onnx(self) -> int:
        for code, member in _ONNX_CODES.items():
            if member is self:
                return code
        return 0


_ONNX_CODES = {
    0: ONNSType.UNDEFINED, 1: ONNSType.FLOAT, 2: ONNSType.UINT8, 3: ONNSType.INT8,
    4: ONNSType.UINT16, 5: ONNSType.INT16, 6: ONNSType.INT32, 7: ONNSType.INT64,
    8: ONNSType.STRING, 9: ONNSType.BOOL, 10: ONNSType.FLOAT16, 11: ONNSType.DOUBLE,
    12: ONNSType.UINT32, 13: ONNSType.UINT64, 16: ONNSType.BFLOAT16,
}

ELEMENT_BYTES = {
    ONNSType.FLOAT: 4, ONNSType.FLOAT16: 2, ONNSType.BFLOAT16: 2, ONNSType.DOUBLE: 8,
    ONNSType.INT8: 1, ONNSType.INT16: 2, ONNSType.INT32: 4, ONNSType.INT64: 8,
    ONNSType.UINT8: 1, ONNSType.UINT16: 2, ONNSType.UINT32: 4, ONNSType.UINT64: 8,
    ONNSType.BOOL: 1,
}


@dataclass
class Tensor:
    name: str
    dtype: ONNSType = ONNSType.UNDEFINED
    shape: List[Any] = field(default_factory=list)
    is_initializer: bool = False
    is_constant: bool = False

    def size_bytes(self) -> Optional[int]:
        """Byte size when every dim is concrete, else None (graph.py:64-95)."""
        if not self.shape:
            return None
        try:
            dims = [int(d) for d in self.shape]
        except (TypeError, ValueError):
            return None
        return ELEMENT_BYTES.get(self.dtype, 4) * math.prod(dims)


@dataclass
class Node:
    id: str
    name: str
    op_type: str
    inputs: List[str] = field(default_factory=list)
    outputs: List[str] = field(default_factory=list)
    attributes: Dict[str, Any] = field(default_factory=dict)
    domain: str = ""


@dataclass
class Edge:
    src_node: str
    dst_node: str
    tensor: str


class Graph:
    """Computation graph with producer/consumer maps and a topological order."""

    def __init__(self) -> None:
        self.name: str = ""
        self.opsets: Dict[str, int] = {}
        self.nodes: Dict[str, Node] = {}
        self.tensors: Dict[str, Tensor] = {}
        self.inputs: List[Tensor] = []
        self.outputs: List[Tensor] = []
        self.initializers: Dict[str, Tensor] = {}
        self.node_order: List[str] = []
        self.tensor_producer: Dict[str, str] = {}
        self.tensor_consumers: Dict[str, List[str]] = {}

    # -- construction -------------------------------------------------------
    def add_node(self, node: Node) -> None:
        self.nodes[node.id] = node
        for name in node.inputs:
            if name:
                self.add_consumer(name, node.id)

    def get_tensor(self, name: str) -> Optional[Tensor]:
        return self.tensors.get(name)

    def register_tensor(self, name: str, dtype: ONNSType = ONNSType.UNDEFINED,
                        shape: Optional[List[Any]] = None, is_initializer: bool = False,
                        is_constant: bool = False) -> Tensor:
        """Create a tensor or update the known fields of an existing one."""
        tensor = self.tensors.get(name)
        if tensor is None:
            tensor = Tensor(name, dtype, [] if shape is None else shape, is_initializer, is_constant)
            self.tensors[name] = tensor
            return tensor
        if dtype != ONNSType.UNDEFINED:
            tensor.dtype = dtype
        if shape is not None:
            tensor.shape = shape
        tensor.is_initializer = tensor.is_initializer or is_initializer
        tensor.is_constant = tensor.is_constant or is_constant
        return tensor

    def set_producer(self, tensor_name: str, node_id: str) -> None:
        current = self.tensor_producer.get(tensor_name)
        if current is not None and current != node_id:
            raise ValueError(
                f"Tensor '{tensor_name}' already has producer '{current}', cannot set to '{node_id}'"
            )
        self.tensor_producer[tensor_name] = node_id

    def add_consumer(self, tensor_name: str, node_id: str) -> None:
        consumers = self.tensor_consumers.setdefault(tensor_name, [])
        if node_id not in consumers:
            consumers.append(node_id)

    # -- ordering -----------------------------------------------------------
    def _successors(self) -> Dict[str, List[str]]:
        succ: Dict[str, List[str]] = {nid: [] for nid in self.nodes}
        for tensor_name, consumers in self.tensor_consumers.items():
            producer = self.tensor_producer.get(tensor_name)
            if producer is None or producer in SPECIAL_PRODUCERS or producer not in self.nodes:
                continue
            for consumer in consumers:
                if consumer in self.nodes:
                    succ[producer].append(consumer)
        return succ

    def topological_sort(self) -> List[str]:
        """Kahn's algorithm; among ready nodes the smallest id goes first."""
        succ = self._successors()
        indegree = {nid: 0 for nid in self.nodes}
        for targets in succ.values():
            for t in targets:
                indegree[t] += 1
        ready = [nid for nid, d in indegree.items() if d == 0]
        heapq.heapify(ready)
        order: List[str] = []
        while ready:
            nid = heapq.heappop(ready)
            order.append(nid)
            for t in succ[nid]:
                indegree[t] -= 1
                if indegree[t] == 0:
                    heapq.heappush(ready, t)
        if len(order) != len(self.nodes):
            stuck = sorted(set(self.nodes) - set(order))
            raise ValueError(f"Graph contains a cycle involving {len(stuck)} nodes: {stuck[:10]}...")
        self.node_order = order
        return order

    def build_edges(self) -> List[Edge]:
        edges = [
            Edge(self.tensor_producer[t], c, t)
            for t, consumers in self.tensor_consumers.items()
            if self.tensor_producer.get(t) in self.nodes
            for c in consumers if c in self.nodes
        ]
        edges.sort(key=lambda e: (e.src_node, e.dst_node, e.tensor))
        return edges

    # -- validation -----------------------------------------------------------
    def validate(self) -> None:
        """Structural checks (graph.py:254-311); also drops dead tensors."""
        for node_id, node in self.nodes.items():
            for name in node.inputs:
                if not name:
                    continue
                if name not in self.tensors:
                    raise ValueError(f"Node '{node_id}' input '{name}' is not a registered tensor")
                producer = self.tensor_producer.get(name)
                if producer is None:
                    raise ValueError(f"Node '{node_id}' input '{name}' has no producer")
                if producer not in SPECIAL_PRODUCERS:
                    pnode = self.nodes.get(producer)
                    if pnode is None or name not in pnode.outputs:
                        raise ValueError(f"Node '{node_id}' input '{name}' has invalid producer '{producer}'")
                if node_id not in self.tensor_consumers.get(name, []):
                    raise ValueError(f"Node '{node_id}' input '{name}' is missing its consumer index")
        dead: List[str] = []
        for name, consumers in self.tensor_consumers.items():
            producer = self.tensor_producer.get(name)
            live = [c for c in consumers if c in self.nodes]
            if producer is None:
                if live:
                    raise ValueError(f"Tensor '{name}' has consumers but no producer")
                dead.append(name)
                continue
            if producer not in SPECIAL_PRODUCERS:
                pnode = self.nodes.get(producer)
                if pnode is None:
                    raise ValueError(f"Tensor '{name}' refers to missing producer '{producer}'")
                if name not in pnode.outputs:
                    raise ValueError(f"Tensor '{name}' claimed producer '{producer}' does not list it as output")
            for c in live:
                if name not in self.nodes[c].inputs:
                    raise ValueError(f"Tensor '{name}' has invalid consumer '{c}'")
        for name in dead:
            self.remove_tensor(name)
        for out in self.outputs:
            if out.name not in self.tensors:
                raise ValueError(f"Graph output '{out.name}' is not a registered tensor")
            if self.tensor_producer.get(out.name) is None:
                raise ValueError(f"Graph output '{out.name}' has no producer")
        self.topological_sort()

    # -- rewriting ------------------------------------------------------------
    def remove_node(self, node_id: str) -> None:
        node = self.nodes.get(node_id)
        if node is None:
            return
        for name in node.inputs:
            consumers = self.tensor_consumers.get(name) if name else None
            if consumers and node_id in consumers:
                consumers.remove(node_id)
        for name in node.outputs:
            if name and self.tensor_producer.get(name) == node_id:
                del self.tensor_producer[name]
        if node_id in self.node_order:
            self.node_order.remove(node_id)
        del self.nodes[node_id]

    def remove_tensor(self, tensor_name: str) -> None:
        if tensor_name not in self.tensors:
            return
        del self.tensors[tensor_name]
        self.tensor_producer.pop(tensor_name, None)
        self.tensor_consumers.pop(tensor_name, None)
        self.initializers.pop(tensor_name, None)

    def replace_node_outputs(self, node_id: str, old_outputs: List[str], new_outputs: List[str]) -> None:
        node = self.nodes[node_id]
        for name in node.outputs:
            if self.tensor_producer.get(name) == node_id:
                del self.tensor_producer[name]
        node.outputs = list(new_outputs)
        for name in new_outputs:
            if name not in self.tensors:
                self.register_tensor(name)
            self.tensor_producer[name] = node_id

    def replace_node_inputs(self, node_id: str, old_inputs: List[str], new_inputs: List[str]) -> None:
        node = self.nodes[node_id]
        for name in node.inputs:
            consumers = self.tensor_consumers.get(name) if name else None
            if consumers and node_id in consumers:
                consumers.remove(node_id)
        node.inputs = list(new_inputs)
        for name in new_inputs:
            if name:
                if name not in self.tensors:
                    self.register_tensor(name)
                self.add_consumer(name, node_id)

    def reroute_consumers(self, old_tensor: str, new_tensor: str) -> None:
        """Point every consumer of old_tensor at new_tensor (no-op if equal)."""
        if old_tensor == new_tensor or old_tensor not in self.tensor_consumers:
            return
        for consumer_id in list(self.tensor_consumers[old_tensor]):
            node = self.nodes.get(consumer_id)
            if node is None:
                continue
            rewired = [new_tensor if name == old_tensor else name for name in node.inputs]
            self.replace_node_inputs(consumer_id, node.inputs, rewired)
            self.add_consumer(new_tensor, consumer_id)
        self.tensor_consumers.pop(old_tensor, None)

    def copy_node_metadata(self, source_id: str, target_id: str) -> None:
        if source_id not in self.nodes or target_id not in self.nodes:
            return
        src, dst = self.nodes[source_id], self.nodes[target_id]
        dst.attributes = dict(src.attributes)
        dst.domain = src.domain
        if src.name and not dst.name:
            dst.name = src.name

    # -- export -----------------------------------------------------------------
    def _display_name(self, node_id: str) -> str:
        node = self.nodes[node_id]
        if not node.name:
            return node_id
        clash = any(n.name == node.name for nid, n in self.nodes.items() if nid != node_id)
        return node_id if clash else node.name

    @staticmethod
    def _shape_json(shape: List[Any]) -> list:
        out = []
        for d in shape:
            try:
                out.append(int(d))
            except (TypeError, ValueError):
                out.append(d)
        return out

    def to_dag_json(self) -> dict:
        if not self.node_order:
            self.topological_sort()
        nodes = []
        for nid in self.node_order:
            node = self.nodes[nid]
            entry: Dict[str, Any] = {"name": self._display_name(nid), "op_type": node.op_type,
                                     "inputs": list(node.inputs), "outputs": list(node.outputs)}
            if node.name and entry["name"] != node.name:
                entry["original_name"] = node.name
            if node.attributes:
                entry["attributes"] = dict(node.attributes)
            nodes.append(entry)
        return {
            "format_version": "1.0",
            "graph_inputs": [{"name": t.name, "dtype": t.dtype.value, "shape": self._shape_json(t.shape)}
                             for t in self.inputs],
            "graph_outputs": [{"name": t.name, "dtype": t.dtype.value, "shape": self._shape_json(t.shape)}
                              for t in self.outputs],
            "nodes": nodes,
            "edges": [{"src_node": self._display_name(e.src_node), "dst_node": self._display_name(e.dst_node),
                       "tensor": e.tensor} for e in self.build_edges()],
        }


def generate_node_id(name: str, op_type: str, idx: int) -> str:
    return name if name else f"_{op_type}_{idx}"
