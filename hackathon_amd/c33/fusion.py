"""Graph fusion passes (counterpart of c33/fusion.py).

Each pass scans the graph in topological order, rewrites matched regions into
one fused node and appends a log record.  The match guards and the fused-node
attribute ABI that the kernels consume (`_flatten_axis`, `_activation`,
`_residual_input_index`, `_ops`, `bn_epsilon` / `bn_parameter_offset`,
`axis` / `epsilon`, `perm` / `allowzero`) follow the reference passes
(c33/fusion.py:174-1455) so the same graphs fuse the same way.
"""

from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Set

from ..c3common.ir.graph import Graph, Node

ELEMENTWISE_OPS: Set[str] = {"Add", "Sub", "Mul", "Div", "Relu", "Erf", "Sqrt", "Exp"}
ELEMENTWISE_ARITH_OPS: Set[str] = {"Add", "Sub", "Mul", "Div"}
MAX_EW_CHAIN = 5


# -- helpers ---------------------------------------------------------------------
def _is_initializer_or_constant(graph: Graph, name: str) -> bool:
    t = graph.tensors.get(name)
    return bool(t is not None and (t.is_initializer or t.is_constant))


def _is_graph_output(graph: Graph, name: str) -> bool:
    return any(t.name == name for t in graph.outputs)


def _dim_compatible(lhs: Any, rhs: Any) -> bool:
    if lhs is None or rhs is None:
        return True
    try:
        return int(lhs) == int(rhs)
    except (TypeError, ValueError):
        return str(lhs) == str(rhs)


def _consumers(graph: Graph, name: str) -> List[str]:
    return [c for c in graph.tensor_consumers.get(name, []) if c in graph.nodes]


def _has_single_consumer(graph: Graph, name: str) -> bool:
    return len(_consumers(graph, name)) == 1


def _only_output(node: Node) -> Optional[str]:
    outs = [o for o in node.outputs if o]
    return outs[0] if len(outs) == 1 else None


def _is_bias_shape(graph: Graph, name: str, output_name: str = "") -> bool:
    """A channel vector (or [1,...,1,C]) matching the output's last dim."""
    t = graph.tensors.get(name)
    if t is None or not t.shape:
        return False
    for d in t.shape[:-1]:
        try:
            if int(d) != 1:
                return False
        except (TypeError, ValueError):
            return False
    out = graph.tensors.get(output_name) if output_name else None
    if out is not None and out.shape and not _dim_compatible(t.shape[-1], out.shape[-1]):
        return False
    return True


def _shapes_maybe_equal(lhs: List[Any], rhs: List[Any]) -> bool:
    if not lhs or not rhs or len(lhs) != len(rhs):
        return False
    for a, b in zip(lhs, rhs):
        try:
            if int(a) != int(b):
                return False
        except (TypeError, ValueError):
            continue
    return True


def _is_dropout_inference(node: Node) -> bool:
    if node.attributes.get("training_mode", 0) not in (0, False, None):
        return False
    return not (len(node.inputs) >= 3 and node.inputs[2])


def _generate_fused_node_id(pattern: str, *parts: str) -> str:
    return f"_{pattern}_{'_'.join(parts)}"


def _unique_fused_node_id(graph: Graph, pattern: str, *parts: str) -> str:
    base = _generate_fused_node_id(pattern, *parts)
    fid, k = base, 1
    while fid in graph.nodes:
        fid, k = f"{base}_{k}", k + 1
    return fid


def _log(log: List[Dict[str, Any]], pattern: str, status: str, old: List[str], new: str = "",
         removed: Optional[List[str]] = None, reason: str = "") -> None:
    log.append({"pattern": pattern, "status": status, "old_node_ids": list(old), "new_node_id": new,
                "removed_tensors": list(removed or []), "rejection_reason": reason})


def _replace_region(graph: Graph, old_ids: List[str], fused: Node) -> List[str]:
    """Swap `old_ids` for `fused`, keeping the fused node's output names."""
    keep = {o for o in fused.outputs if o}
    removed = sorted({o for nid in old_ids for o in graph.nodes[nid].outputs if o and o not in keep})
    for nid in reversed(old_ids):
        graph.remove_node(nid)
    graph.add_node(fused)
    for o in fused.outputs:
        if o:
            if o not in graph.tensors:
                graph.register_tensor(o)
            graph.set_producer(o, fused.id)
    return removed


def _fuse_pair(graph: Graph, first: Node, second: Node, fused: Node) -> List[str]:
    """Replace a producer->consumer pair whose consumer outputs survive."""
    for o in second.outputs:
        if o:
            graph.tensor_producer.pop(o, None)
    graph.add_node(fused)
    for o in fused.outputs:
        if o:
            if o not in graph.tensors:
                graph.register_tensor(o)
            graph.set_producer(o, fused.id)
    removed = [t for t in list(first.outputs) + list(second.outputs) if t and t in graph.tensors]
    graph.remove_node(second.id)
    graph.remove_node(first.id)
    return removed


# -- F1a MatMul -> Add(bias) -------------------------------------------------------
def fuse_matmul_bias(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    fusions, done = 0, set()
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if nid in done or node is None or node.op_type != "MatMul":
            continue
        pattern = "FusedMatMulBias"
        w = graph.tensors.get(node.inputs[1]) if len(node.inputs) >= 2 else None
        if len(node.inputs) < 2:
            continue
        if w is None or len(w.shape) != 2:
            _log(fusion_log, pattern, "skipped", [nid], reason="Single-kernel epilogue requires rank-2 B")
            continue
        mm_out = _only_output(node)
        if mm_out is None:
            continue
        if _is_graph_output(graph, mm_out):
            _log(fusion_log, pattern, "skipped", [nid], reason="MatMul output is an observable graph output")
            continue
        if not _has_single_consumer(graph, mm_out):
            _log(fusion_log, pattern, "skipped", [nid], reason="MatMul output has multiple consumers")
            continue
        add = graph.nodes.get(_consumers(graph, mm_out)[0])
        if add is None or add.op_type != "Add":
            continue
        add_in = [i for i in add.inputs if i]
        if len(add_in) != 2:
            continue
        bias = next((i for i in add_in if i != mm_out), None)
        if bias is None:
            continue
        if not _is_initializer_or_constant(graph, bias) or not _is_bias_shape(graph, bias, mm_out):
            _log(fusion_log, pattern, "skipped", [nid, add.id],
                 reason="Bias input is not a compatible initializer/constant")
            continue
        fid = _generate_fused_node_id(pattern, nid, add.id)
        fused = Node(id=fid, name=f"fused_matmul_bias_{nid}_{add.id}", op_type=pattern,
                     inputs=[i for i in node.inputs if i] + [bias], outputs=list(add.outputs),
                     attributes=dict(node.attributes))
        add_out = _only_output(add)
        removed = [t for t in list(node.outputs) + list(add.outputs) if t and t in graph.tensors]
        for o in add.outputs:
            if o:
                graph.tensor_producer.pop(o, None)
        graph.add_node(fused)
        for o in fused.outputs:
            if o:
                if o not in graph.tensors:
                    graph.register_tensor(o)
                graph.set_producer(o, fid)
        if add_out:
            graph.reroute_consumers(add_out, fused.outputs[0])
            for t in graph.outputs:
                if t.name == add_out:
                    t.name = fused.outputs[0]
        graph.reroute_consumers(mm_out, fused.outputs[0])
        graph.remove_node(add.id)
        graph.remove_node(nid)
        done.update({nid, add.id})
        fusions += 1
        _log(fusion_log, pattern, "fused", [nid, add.id], fid, removed)
    return fusions


# -- F1b Conv -> BatchNormalization -------------------------------------------------
def fuse_conv_batchnorm(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    fusions, done = 0, set()
    pattern = "FusedConv2dBatchNorm"
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if nid in done or node is None or node.op_type != "Conv":
            continue
        conv_out = _only_output(node)
        if conv_out is None:
            continue
        if _is_graph_output(graph, conv_out):
            _log(fusion_log, pattern, "skipped", [nid], reason="Conv output is an observable graph output")
            continue
        if not _has_single_consumer(graph, conv_out):
            _log(fusion_log, pattern, "skipped", [nid],
                 reason="Conv output has multiple consumers, cannot safely fuse")
            continue
        bn = graph.nodes.get(_consumers(graph, conv_out)[0])
        if bn is None or bn.op_type not in ("BatchNormalization", "BatchNorm"):
            continue
        pair = [nid, bn.id]
        if _only_output(bn) is None:
            _log(fusion_log, pattern, "skipped", pair, reason="BatchNormalization has observable auxiliary outputs")
            continue
        bn_in = [i for i in bn.inputs if i]
        if len(bn_in) < 5:
            _log(fusion_log, pattern, "skipped", pair,
                 reason="BatchNormalization missing required parameters (need 5 inputs)")
            continue
        params = bn_in[1:5]
        if not all(_is_initializer_or_constant(graph, p) for p in params):
            _log(fusion_log, pattern, "skipped", pair,
                 reason="BN parameters are not initializers/constants, cannot fold")
            continue
        w = graph.tensors.get(node.inputs[1]) if len(node.inputs) > 1 else None
        channels = w.shape[0] if w is not None and w.shape else None
        if channels is not None:
            bad = [p for p in params if graph.tensors.get(p) is None or len(graph.tensors[p].shape) != 1
                   or not _dim_compatible(graph.tensors[p].shape[0], channels)]
            if bad:
                _log(fusion_log, pattern, "skipped", pair, reason="BN parameter shape does not match Conv channels")
                continue
        attrs = dict(node.attributes)
        attrs["bn_epsilon"] = bn.attributes.get("epsilon", 1e-5)
        attrs["bn_parameter_offset"] = len(node.inputs)
        fid = _generate_fused_node_id(pattern, nid, bn.id)
        fused = Node(id=fid, name=f"fused_conv_bn_{nid}_{bn.id}", op_type=pattern,
                     inputs=list(node.inputs) + params, outputs=list(bn.outputs), attributes=attrs)
        bn_out = _only_output(bn)
        removed = _fuse_pair(graph, node, bn, fused)
        graph.reroute_consumers(bn_out, fused.outputs[0])
        for t in graph.outputs:
            if t.name == bn_out:
                t.name = fused.outputs[0]
        done.update(pair)
        fusions += 1
        _log(fusion_log, pattern, "fused", pair, fid, removed)
    return fusions


# -- F1c elementwise chains ------------------------------------------------------------
def _walk_elementwise_chain(graph: Graph, start: str, visited: Set[str]) -> List[str]:
    chain = [start]
    outputs = {t.name for t in graph.outputs}
    cur = start
    while len(chain) < MAX_EW_CHAIN:
        node = graph.nodes.get(cur)
        out = _only_output(node) if node is not None else None
        if out is None or out in outputs:
            break
        consumers = _consumers(graph, out)
        if len(consumers) != 1 or consumers[0] in visited:
            break
        nxt = graph.nodes.get(consumers[0])
        if nxt is None or nxt.op_type not in ELEMENTWISE_OPS:
            break
        chain.append(nxt.id)
        visited.add(nxt.id)
        cur = nxt.id
    return chain


def fuse_elementwise_chain(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    """2-5 single-consumer elementwise nodes -> FusedEWChain with an `_ops` program."""
    fusions, visited = 0, set()
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if nid in visited or node is None or node.op_type not in ELEMENTWISE_OPS:
            continue
        chain = _walk_elementwise_chain(graph, nid, visited)
        if len(chain) < 2:
            visited.update(chain)
            continue
        nodes = [graph.nodes[c] for c in chain]
        ops = [n.op_type for n in nodes]
        internal = {o for n in nodes for o in n.outputs if o}
        inputs: List[str] = []
        for n in nodes:
            for i in n.inputs:
                if i and i not in internal and i not in inputs:
                    inputs.append(i)
        index = {name: k for k, name in enumerate(inputs)}
        program = [{"op": n.op_type, "attrs": dict(n.attributes),
                    "inputs": [i if i in internal else index[i] for i in n.inputs if i],
                    "output": next((o for o in n.outputs if o), "")} for n in nodes]
        fid = _generate_fused_node_id("FusedEWChain", "_".join(ops), chain[0])
        last = nodes[-1]
        for o in last.outputs:
            if o:
                graph.tensor_producer.pop(o, None)
        fused = Node(id=fid, name=f"fused_ew_chain_{'_'.join(ops)}_{chain[0]}", op_type="FusedEWChain",
                     inputs=inputs, outputs=list(last.outputs),
                     attributes={"chain_ops": ops, "chain_node_ids": list(chain), "_ops": program})
        graph.add_node(fused)
        for o in fused.outputs:
            if o:
                if o not in graph.tensors:
                    graph.register_tensor(o)
                graph.set_producer(o, fid)
        last_out = _only_output(last)
        if last_out:
            graph.reroute_consumers(last_out, fused.outputs[0])
            for t in graph.outputs:
                if t.name == last_out:
                    t.name = fused.outputs[0]
        removed = [o for c in chain for o in graph.nodes[c].outputs if o and o in graph.tensors]
        for c in chain:
            graph.remove_node(c)
            visited.add(c)
        fusions += 1
        _log(fusion_log, "FusedEWChain", "fused", chain, fid, removed)
    return fusions


# -- F1d Softmax -> Dropout(inference) --------------------------------------------------
def fuse_softmax_dropout(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    fusions, done = 0, set()
    pattern = "FusedSoftmaxDropout"
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if nid in done or node is None or node.op_type != "Softmax":
            continue
        out = _only_output(node)
        if out is None:
            continue
        if _is_graph_output(graph, out):
            _log(fusion_log, pattern, "skipped", [nid], reason="Softmax output is an observable graph output")
            continue
        if not _has_single_consumer(graph, out):
            _log(fusion_log, pattern, "skipped", [nid], reason="Softmax output has multiple consumers")
            continue
        drop = graph.nodes.get(_consumers(graph, out)[0])
        if drop is None or drop.op_type != "Dropout":
            continue
        pair = [nid, drop.id]
        if _only_output(drop) is None:
            _log(fusion_log, pattern, "skipped", pair, reason="Dropout mask output is observable")
            continue
        if not _is_dropout_inference(drop):
            _log(fusion_log, pattern, "skipped", pair, reason="Dropout is in training mode, inference-only fusion")
            continue
        attrs = dict(node.attributes)
        attrs["dropout_ratio"] = drop.attributes.get("ratio", 0.0)
        fid = _generate_fused_node_id(pattern, nid, drop.id)
        fused = Node(id=fid, name=f"fused_softmax_dropout_{nid}_{drop.id}", op_type=pattern,
                     inputs=list(node.inputs), outputs=list(drop.outputs), attributes=attrs)
        drop_out = _only_output(drop)
        removed = _fuse_pair(graph, node, drop, fused)
        graph.reroute_consumers(drop_out, fused.outputs[0])
        for t in graph.outputs:
            if t.name == drop_out:
                t.name = fused.outputs[0]
        done.update(pair)
        fusions += 1
        _log(fusion_log, pattern, "fused", pair, fid, removed)
    return fusions


# -- F1e residual Add -> LayerNormalization ------------------------------------------------
def fuse_residual_norm(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    fusions, done = 0, set()
    pattern = "FusedResidualNorm"
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if nid in done or node is None or node.op_type != "Add":
            continue
        ins = [i for i in node.inputs if i]
        if len(ins) != 2 or any(_is_initializer_or_constant(graph, i) for i in ins):
            continue
        left, right = graph.tensors.get(ins[0]), graph.tensors.get(ins[1])
        if (left is not None and right is not None and left.shape and right.shape and
                (len(left.shape) != len(right.shape)
                 or not all(_dim_compatible(a, b) for a, b in zip(left.shape, right.shape)))):
            continue
        out = _only_output(node)
        if out is None:
            continue
        if _is_graph_output(graph, out):
            _log(fusion_log, pattern, "skipped", [nid], reason="Residual Add output is an observable graph output")
            continue
        if not _has_single_consumer(graph, out):
            _log(fusion_log, pattern, "skipped", [nid],
                 reason="Add output has multiple consumers, cannot safely fuse with LayerNorm")
            continue
        ln = graph.nodes.get(_consumers(graph, out)[0])
        if ln is None or ln.op_type not in ("LayerNormalization", "LayerNorm"):
            continue
        pair = [nid, ln.id]
        if _only_output(ln) is None:
            _log(fusion_log, pattern, "skipped", pair, reason="LayerNormalization has observable auxiliary outputs")
            continue
        try:
            axis = int(ln.attributes.get("axis", -1))
            eps = float(ln.attributes.get("epsilon", 1e-5))
        except (TypeError, ValueError):
            continue
        if not math.isfinite(eps) or eps <= 0.0:
            continue
        ln_in = [i for i in ln.inputs if i]
        scale = ln_in[1] if len(ln_in) > 1 else ""
        bias = ln_in[2] if len(ln_in) > 2 else ""
        if not scale:
            continue
        normalized = graph.tensors.get(out)
        if normalized is not None and normalized.shape:
            rank = len(normalized.shape)
            ax = axis + rank if axis < 0 else axis
            if not 0 <= ax < rank:
                continue
            expect = list(normalized.shape[ax:])
            ok = True
            for p in (scale, bias):
                if not p:
                    continue
                pt = graph.tensors.get(p)
                if pt is None or len(pt.shape) != len(expect) or not all(
                        _dim_compatible(a, b) for a, b in zip(pt.shape, expect)):
                    ok = False
                    break
            if not ok:
                continue
        attrs = dict(node.attributes)
        attrs.update({"ln_axis": axis, "ln_epsilon": eps, "ln_scale": scale, "ln_bias": bias,
                      "axis": axis, "epsilon": eps})
        fid = _generate_fused_node_id(pattern, nid, ln.id)
        fused = Node(id=fid, name=f"fused_residual_norm_{nid}_{ln.id}", op_type=pattern,
                     inputs=list(node.inputs) + [p for p in (scale, bias) if p], outputs=list(ln.outputs),
                     attributes=attrs)
        ln_out = _only_output(ln)
        removed = _fuse_pair(graph, node, ln, fused)
        graph.reroute_consumers(ln_out, fused.outputs[0])
        for t in graph.outputs:
            if t.name == ln_out:
                t.name = fused.outputs[0]
        done.update(pair)
        fusions += 1
        _log(fusion_log, pattern, "fused", pair, fid, removed)
    return fusions


# -- Gemm (+Flatten producer) (+Relu) -> FusedGemmEpilogue -----------------------------------
def fuse_gemm_epilogues(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    if not graph.node_order:
        graph.topological_sort()
    fusions = 0
    for nid in list(graph.node_order):
        gemm = graph.nodes.get(nid)
        if gemm is None or gemm.op_type != "Gemm" or _only_output(gemm) is None:
            continue
        old: List[str] = []
        inputs, attrs = list(gemm.inputs), dict(gemm.attributes)
        if inputs:
            prod = graph.nodes.get(graph.tensor_producer.get(inputs[0]) or "")
            if (prod is not None and prod.op_type == "Flatten" and _only_output(prod) is not None
                    and _has_single_consumer(graph, prod.outputs[0])
                    and not _is_graph_output(graph, prod.outputs[0])):
                attrs["_flatten_axis"] = int(prod.attributes.get("axis", 1))
                inputs[0] = prod.inputs[0]
                old.append(prod.id)
        old.append(gemm.id)
        final = gemm
        out = _only_output(gemm)
        if not _is_graph_output(graph, out) and _has_single_consumer(graph, out):
            relu = graph.nodes.get(_consumers(graph, out)[0])
            if relu is not None and relu.op_type == "Relu" and _only_output(relu) is not None:
                attrs["_activation"] = "Relu"
                final = relu
                old.append(relu.id)
        fid = _unique_fused_node_id(graph, "FusedGemmEpilogue", old[0], old[-1])
        fused = Node(id=fid, name=f"fused_gemm_epilogue_{gemm.id}", op_type="FusedGemmEpilogue",
                     inputs=inputs, outputs=list(final.outputs), attributes=attrs, domain=gemm.domain)
        removed = _replace_region(graph, old, fused)
        _log(fusion_log, "FusedGemmEpilogue", "fused", old, fid, removed)
        fusions += 1
    if fusions:
        graph.topological_sort()
    return fusions


# -- Conv (+Relu | +Add+Relu) -> FusedConv(Residual)Activation --------------------------------
def _preferred_conv_for_add(graph: Graph, add: Node, order: Dict[str, int]) -> Optional[str]:
    """The latest Conv producer feeding the residual Add (main path)."""
    convs = [p for p in (graph.tensor_producer.get(i) for i in add.inputs)
             if p in graph.nodes and graph.nodes[p].op_type == "Conv"]
    return max(convs, key=lambda c: order.get(c, -1)) if convs else None


def fuse_conv_epilogues(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    if not graph.node_order:
        graph.topological_sort()
    order = {nid: i for i, nid in enumerate(graph.node_order)}
    fusions = 0
    for nid in list(graph.node_order):
        conv = graph.nodes.get(nid)
        if conv is None or conv.op_type != "Conv":
            continue
        out = _only_output(conv)
        if out is None or _is_graph_output(graph, out) or not _has_single_consumer(graph, out):
            continue
        consumer = graph.nodes.get(_consumers(graph, out)[0])
        if consumer is None:
            continue
        inputs, attrs = list(conv.inputs), dict(conv.attributes)
        op_type = "FusedConvActivation"
        if consumer.op_type == "Relu":
            old, final = [conv.id, consumer.id], consumer
            attrs["_activation"] = "Relu"
        elif consumer.op_type == "Add" and len(consumer.inputs) == 2:
            if _preferred_conv_for_add(graph, consumer, order) != conv.id:
                continue
            add_out = _only_output(consumer)
            if add_out is None or _is_graph_output(graph, add_out) or not _has_single_consumer(graph, add_out):
                continue
            relu = graph.nodes.get(_consumers(graph, add_out)[0])
            if relu is None or relu.op_type != "Relu":
                continue
            residual = consumer.inputs[1] if consumer.inputs[0] == out else consumer.inputs[0]
            rt = graph.tensors.get(residual)
            if rt is None or not _shapes_maybe_equal(list(graph.tensors[out].shape), list(rt.shape)):
                continue
            attrs["_activation"] = "Relu"
            attrs["_residual_input_index"] = len(inputs)
            inputs.append(residual)
            old, final, op_type = [conv.id, consumer.id, relu.id], relu, "FusedConvResidualActivation"
        else:
            continue
        fid = _unique_fused_node_id(graph, op_type, old[0], old[-1])
        fused = Node(id=fid, name=f"fused_conv_epilogue_{conv.id}", op_type=op_type, inputs=inputs,
                     outputs=list(final.outputs), attributes=attrs, domain=conv.domain)
        removed = _replace_region(graph, old, fused)
        _log(fusion_log, op_type, "fused", old, fid, removed)
        fusions += 1
    if fusions:
        graph.topological_sort()
    return fusions


# -- MatMul(rank 4) -> Div -> Add(mask) -> Softmax -> FusedAttentionScores ----------------------
def fuse_attention_scores(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    if not graph.node_order:
        graph.topological_sort()
    fusions = 0
    for nid in list(graph.node_order):
        mm = graph.nodes.get(nid)
        if mm is None or mm.op_type != "MatMul" or len(mm.inputs) != 2:
            continue
        out = _only_output(mm)
        if out is None or _is_graph_output(graph, out):
            continue
        lhs, rhs, res = (graph.tensors.get(n) for n in (mm.inputs[0], mm.inputs[1], out))
        if (lhs is None or rhs is None or res is None or len(lhs.shape) != 4 or len(rhs.shape) != 4
                or len(res.shape) != 4 or not _has_single_consumer(graph, out)):
            continue
        div = graph.nodes.get(_consumers(graph, out)[0])
        if (div is None or div.op_type != "Div" or len(div.inputs) != 2 or div.inputs[0] != out
                or _only_output(div) is None):
            continue
        divisor = graph.tensors.get(div.inputs[1])
        if divisor is None or len(divisor.shape) > 1:
            continue
        div_out = _only_output(div)
        if _is_graph_output(graph, div_out) or not _has_single_consumer(graph, div_out):
            continue
        add = graph.nodes.get(_consumers(graph, div_out)[0])
        if add is None or add.op_type != "Add" or len(add.inputs) != 2:
            continue
        mask_name = add.inputs[1] if add.inputs[0] == div_out else add.inputs[0]
        mask = graph.tensors.get(mask_name)
        add_out = _only_output(add)
        if (mask is None or len(mask.shape) > 4 or add_out is None or _is_graph_output(graph, add_out)
                or not _has_single_consumer(graph, add_out)):
            continue
        sm = graph.nodes.get(_consumers(graph, add_out)[0])
        if sm is None or sm.op_type != "Softmax" or int(sm.attributes.get("axis", -1)) not in (-1, 3):
            continue
        fid = _unique_fused_node_id(graph, "FusedAttentionScores", mm.id, sm.id)
        fused = Node(id=fid, name=f"fused_attention_scores_{mm.id}", op_type="FusedAttentionScores",
                     inputs=[mm.inputs[0], mm.inputs[1], div.inputs[1], mask_name], outputs=list(sm.outputs),
                     attributes={"axis": -1}, domain=mm.domain)
        old = [mm.id, div.id, add.id, sm.id]
        removed = _replace_region(graph, old, fused)
        _log(fusion_log, "FusedAttentionScores", "fused", old, fid, removed)
        fusions += 1
    if fusions:
        graph.topological_sort()
    return fusions


# -- Transpose -> Reshape -> FusedTransposeReshape --------------------------------------------
def fuse_transpose_reshape(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    if not graph.node_order:
        graph.topological_sort()
    fusions = 0
    for nid in list(graph.node_order):
        tr = graph.nodes.get(nid)
        if tr is None or tr.op_type != "Transpose":
            continue
        out = _only_output(tr)
        if out is None or _is_graph_output(graph, out) or not _has_single_consumer(graph, out):
            continue
        src = graph.tensors.get(tr.inputs[0])
        if src is None or not 1 <= len(src.shape) <= 4:
            continue
        rs = graph.nodes.get(_consumers(graph, out)[0])
        if rs is None or rs.op_type != "Reshape" or len(rs.inputs) < 2 or _only_output(rs) is None:
            continue
        perm_attr = tr.attributes.get("perm")
        perm = list(range(len(src.shape) - 1, -1, -1)) if perm_attr is None else [int(v) for v in perm_attr]
        if sorted(perm) != list(range(len(src.shape))):
            continue
        fid = _unique_fused_node_id(graph, "FusedTransposeReshape", tr.id, rs.id)
        fused = Node(id=fid, name=f"fused_transpose_reshape_{tr.id}", op_type="FusedTransposeReshape",
                     inputs=[tr.inputs[0], rs.inputs[1]], outputs=list(rs.outputs),
                     attributes={"perm": perm, "allowzero": int(rs.attributes.get("allowzero", 0))},
                     domain=tr.domain)
        old = [tr.id, rs.id]
        removed = _replace_region(graph, old, fused)
        _log(fusion_log, "FusedTransposeReshape", "fused", old, fid, removed)
        fusions += 1
    if fusions:
        graph.topological_sort()
    return fusions


# -- single-output LayerNormalization -> FusedLayerNormalization ----------------------------------
def fuse_layer_normalization_kernels(graph: Graph, fusion_log: List[Dict[str, Any]]) -> int:
    fusions = 0
    for nid in list(graph.node_order):
        node = graph.nodes.get(nid)
        if node is None or node.op_type not in ("LayerNormalization", "LayerNorm") or _only_output(node) is None:
            continue
        fid = _unique_fused_node_id(graph, "FusedLayerNormalization", node.id)
        fused = Node(id=fid, name=f"fused_layer_normalization_{node.id}", op_type="FusedLayerNormalization",
                     inputs=list(node.inputs), outputs=list(node.outputs), attributes=dict(node.attributes),
                     domain=node.domain)
        removed = _replace_region(graph, [node.id], fused)
        _log(fusion_log, "FusedLayerNormalization", "fused", [node.id], fid, removed)
        fusions += 1
    if fusions:
        graph.topological_sort()
    return fusions


def cleanup_dead_tensors(graph: Graph) -> int:
    removed = 0
    inputs = {t.name for t in graph.inputs}
    outputs = {t.name for t in graph.outputs}
    for name in list(graph.tensors):
        t = graph.tensors.get(name)
        if t is None or name in inputs or name in outputs or t.is_initializer or t.is_constant:
            continue
        prod = graph.tensor_producer.get(name)
        has_prod = prod is not None and (prod in ("INPUT", "INITIALIZER", "CONSTANT") or prod in graph.nodes)
        if not has_prod and not _consumers(graph, name):
            graph.remove_tensor(name)
            removed += 1
    return removed
