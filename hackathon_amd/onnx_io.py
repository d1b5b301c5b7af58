"""ONNX wire format without the `onnx` package: read, write, import to the IR.

The ONNX protobuf schema (onnx.proto, opset-independent) is declared here as a
hand-built proto2 FileDescriptorProto with the official field numbers, so
`google.protobuf` can parse and serialize `.onnx` files on machines where the
`onnx` package is absent.  On top of it:

* `import_onnx(path)` builds the C3 IR `Graph` with the semantics of
  c31/import_onnx.py:60-200 (initializers registered as tensors, graph inputs
  minus initializers, outputs, value_info, deterministic node ids with
  duplicate suffixes, optional-input positions kept, Constant outputs typed),
  and fills shapes the file leaves open with `infer_shapes` (the op subset of
  the C3 path), which the reference delegated to onnx.shape_inference.
* `read_initializers_and_constants(path)` returns host arrays for
  initializers and Constant outputs (c35/executor.py:23-88).
* `export_model(graph, weights, path)` writes a Graph + weights as a valid
  ModelProto (raw_data tensors, value_info for every known shape).
"""

from __future__ import annotations

import base64
import math
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
from google.protobuf import descriptor_pb2, descriptor_pool, message_factory
from google.protobuf.json_format import MessageToDict
from google.protobuf.message import Message

from .c3common.ir.graph import Graph, Node, ONNSType, generate_node_id

# ------------------------------------------------------------------ schema
_F = descriptor_pb2.FieldDescriptorProto
_OPT, _REP = _F.LABEL_OPTIONAL, _F.LABEL_REPEATED
_T = {"int64": _F.TYPE_INT64, "int32": _F.TYPE_INT32, "uint64": _F.TYPE_UINT64, "float": _F.TYPE_FLOAT,
      "double": _F.TYPE_DOUBLE, "string": _F.TYPE_STRING, "bytes": _F.TYPE_BYTES, "msg": _F.TYPE_MESSAGE,
      "enum": _F.TYPE_ENUM}

# (message, [(field name, number, label, type, type_name or None, packed)])
_SCHEMA: List[Tuple[str, List[Tuple[str, int, int, str, Optional[str], bool]]]] = [
    ("StringStringEntryProto", [("key", 1, _OPT, "string", None, False), ("value", 2, _OPT, "string", None, False)]),
    ("OperatorSetIdProto", [("domain", 1, _OPT, "string", None, False), ("version", 2, _OPT, "int64", None, False)]),
    ("TensorShapeProto.Dimension", [("dim_value", 1, _OPT, "int64", None, False),
                                    ("dim_param", 2, _OPT, "string", None, False),
                                    ("denotation", 3, _OPT, "string", None, False)]),
    ("TensorShapeProto", [("dim", 1, _REP, "msg", ".onnx.TensorShapeProto.Dimension", False)]),
    ("TypeProto.Tensor", [("elem_type", 1, _OPT, "int32", None, False),
                          ("shape", 2, _OPT, "msg", ".onnx.TensorShapeProto", False)]),
    ("TypeProto", [("tensor_type", 1, _OPT, "msg", ".onnx.TypeProto.Tensor", False),
                   ("denotation", 6, _OPT, "string", None, False)]),
    ("ValueInfoProto", [("name", 1, _OPT, "string", None, False), ("type", 2, _OPT, "msg", ".onnx.TypeProto", False),
                        ("doc_string", 3, _OPT, "string", None, False)]),
    ("TensorProto.Segment", [("begin", 1, _OPT, "int64", None, False), ("end", 2, _OPT, "int64", None, False)]),
    ("TensorProto", [("dims", 1, _REP, "int64", None, False), ("data_type", 2, _OPT, "int32", None, False),
                     ("segment", 3, _OPT, "msg", ".onnx.TensorProto.Segment", False),
                     ("float_data", 4, _REP, "float", None, True), ("int32_data", 5, _REP, "int32", None, True),
                     ("string_data", 6, _REP, "bytes", None, False), ("int64_data", 7, _REP, "int64", None, True),
                     ("name", 8, _OPT, "string", None, False), ("raw_data", 9, _OPT, "bytes", None, False),
                     ("double_data", 10, _REP, "double", None, True), ("uint64_data", 11, _REP, "uint64", None, True),
                     ("doc_string", 12, _OPT, "string", None, False),
                     ("external_data", 13, _REP, "msg", ".onnx.StringStringEntryProto", False),
                     ("data_location", 14, _OPT, "int32", None, False)]),
    ("AttributeProto", [("name", 1, _OPT, "string", None, False), ("f", 2, _OPT, "float", None, False),
                        ("i", 3, _OPT, "int64", None, False), ("s", 4, _OPT, "bytes", None, False),
                        ("t", 5, _OPT, "msg", ".onnx.TensorProto", False),
                        ("g", 6, _OPT, "msg", ".onnx.GraphProto", False),
                        ("floats", 7, _REP, "float", None, False), ("ints", 8, _REP, "int64", None, False),
                        ("strings", 9, _REP, "bytes", None, False),
                        ("tensors", 10, _REP, "msg", ".onnx.TensorProto", False),
                        ("graphs", 11, _REP, "msg", ".onnx.GraphProto", False),
                        ("doc_string", 13, _OPT, "string", None, False),
                        ("type", 20, _OPT, "int32", None, False),
                        ("ref_attr_name", 21, _OPT, "string", None, False)]),
    ("NodeProto", [("input", 1, _REP, "string", None, False), ("output", 2, _REP, "string", None, False),
                   ("name", 3, _OPT, "string", None, False), ("op_type", 4, _OPT, "string", None, False),
                   ("attribute", 5, _REP, "msg", ".onnx.AttributeProto", False),
                   ("doc_string", 6, _OPT, "string", None, False), ("domain", 7, _OPT, "string", None, False)]),
    ("GraphProto", [("node", 1, _REP, "msg", ".onnx.NodeProto", False), ("name", 2, _OPT, "string", None, False),
                    ("initializer", 5, _REP, "msg", ".onnx.TensorProto", False),
                    ("doc_string", 10, _OPT, "string", None, False),
                    ("input", 11, _REP, "msg", ".onnx.ValueInfoProto", False),
                    ("output", 12, _REP, "msg", ".onnx.ValueInfoProto", False),
                    ("value_info", 13, _REP, "msg", ".onnx.ValueInfoProto", False)]),
    ("ModelProto", [("ir_version", 1, _OPT, "int64", None, False),
                    ("producer_name", 2, _OPT, "string", None, False),
                    ("producer_version", 3, _OPT, "string", None, False), ("domain", 4, _OPT, "string", None, False),
                    ("model_version", 5, _OPT, "int64", None, False), ("doc_string", 6, _OPT, "string", None, False),
                    ("graph", 7, _OPT, "msg", ".onnx.GraphProto", False),
                    ("opset_import", 8, _REP, "msg", ".onnx.OperatorSetIdProto", False),
                    ("metadata_props", 14, _REP, "msg", ".onnx.StringStringEntryProto", False)]),
]


def _build_classes() -> Dict[str, Any]:
    fd = descriptor_pb2.FileDescriptorProto(name="c3_onnx_subset.proto", package="onnx", syntax="proto2")
    msgs: Dict[str, descriptor_pb2.DescriptorProto] = {}
    for full, fields in sorted(_SCHEMA, key=lambda e: e[0].count(".")):  # parents before nested types
        parts = full.split(".")
        if len(parts) == 1:
            m = fd.message_type.add(name=parts[0])
        else:
            m = msgs[parts[0]].nested_type.add(name=parts[1])
        msgs[full] = m
        for name, num, label, typ, type_name, packed in fields:
            f = m.field.add(name=name, number=num, label=label, type=_T[typ])
            if type_name:
                f.type_name = type_name
            if packed:
                f.options.packed = True
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fd)
    return {full: message_factory.GetMessageClass(pool.FindMessageTypeByName("onnx." + full))
            for full, _ in _SCHEMA}


_CLASSES = _build_classes()
ModelProto = _CLASSES["ModelProto"]
GraphProto = _CLASSES["GraphProto"]
NodeProto = _CLASSES["NodeProto"]
TensorProto = _CLASSES["TensorProto"]
AttributeProto = _CLASSES["AttributeProto"]
ValueInfoProto = _CLASSES["ValueInfoProto"]

# TensorProto.DataType -> numpy (BFLOAT16 is kept as its uint16 bit pattern)
_NP_OF = {1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16, 5: np.int16, 6: np.int32, 7: np.int64,
          9: np.bool_, 10: np.float16, 11: np.float64, 12: np.uint32, 13: np.uint64, 16: np.uint16}
_CODE_OF = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3, np.dtype(np.uint16): 4,
            np.dtype(np.int16): 5, np.dtype(np.int32): 6, np.dtype(np.int64): 7, np.dtype(np.bool_): 9,
            np.dtype(np.float16): 10, np.dtype(np.float64): 11, np.dtype(np.uint32): 12, np.dtype(np.uint64): 13}
# AttributeProto.AttributeType
A_FLOAT, A_INT, A_STRING, A_TENSOR, A_GRAPH, A_FLOATS, A_INTS, A_STRINGS = 1, 2, 3, 4, 5, 6, 7, 8


# ------------------------------------------------------------------ tensors
def tensor_to_numpy(t) -> np.ndarray:
    """TensorProto -> array (raw_data or the typed repeated field)."""
    if t.data_location == 1:
        raise ValueError(f"tensor '{t.name}': external data is not supported")
    dt = _NP_OF.get(t.data_type)
    if dt is None:
        raise ValueError(f"tensor '{t.name}': data_type {t.data_type} unsupported")
    shape = tuple(int(d) for d in t.dims)
    count = math.prod(shape)
    if t.raw_data:
        arr = np.frombuffer(t.raw_data, dtype=np.dtype(dt).newbyteorder("<")).astype(dt)
    elif t.data_type in (1,):
        arr = np.asarray(t.float_data, np.float32)
    elif t.data_type in (11,):
        arr = np.asarray(t.double_data, np.float64)
    elif t.data_type in (7,):
        arr = np.asarray(t.int64_data, np.int64)
    elif t.data_type in (12, 13):
        arr = np.asarray(t.uint64_data, dt)
    elif t.data_type in (10, 16):  # 16-bit values stored in int32_data as bit patterns
        arr = np.asarray(t.int32_data, np.uint16).view(dt)
    else:  # int32_data carries the remaining narrow types
        arr = np.asarray(t.int32_data, np.int64).astype(dt)
    if arr.size != count:
        raise ValueError(f"tensor '{t.name}': {arr.size} values for shape {shape}")
    return arr.reshape(shape)


def numpy_to_tensor(name: str, arr: np.ndarray):
    arr = np.asarray(arr)  # (ascontiguousarray would turn a 0-d scalar into shape (1,))
    code = _CODE_OF.get(arr.dtype)
    if code is None:
        raise ValueError(f"tensor '{name}': dtype {arr.dtype} has no ONNX data type")
    t = TensorProto(name=name, data_type=code)
    t.dims.extend(int(d) for d in arr.shape)
    t.raw_data = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
    return t


# ------------------------------------------------------------------ attributes
def _json_safe(value: Any) -> Any:
    if value is None or isinstance(value, (bool, int, float, str)):
        return value
    if isinstance(value, bytes):
        try:
            return value.decode("utf-8")
        except UnicodeDecodeError:
            return {"base64": base64.b64encode(value).decode("ascii")}
    if isinstance(value, (list, tuple)):
        return [_json_safe(v) for v in value]
    if isinstance(value, Message):
        return MessageToDict(value, preserving_proto_field_name=True)
    return str(value)


def attribute_value(a) -> Any:
    """AttributeProto -> Python value (the subset onnx.helper.get_attribute_value covers here)."""
    kind = a.type
    if kind == 0:  # legacy files without `type`: infer from the populated field
        kind = (A_FLOATS if a.floats else A_INTS if a.ints else A_STRINGS if a.strings else
                A_TENSOR if a.HasField("t") else A_STRING if a.HasField("s") else
                A_FLOAT if a.HasField("f") else A_INT)
    if kind == A_FLOAT:
        return float(a.f)
    if kind == A_INT:
        return int(a.i)
    if kind == A_STRING:
        return a.s
    if kind == A_TENSOR:
        return a.t
    if kind == A_GRAPH:
        return a.g
    if kind == A_FLOATS:
        return [float(v) for v in a.floats]
    if kind == A_INTS:
        return [int(v) for v in a.ints]
    if kind == A_STRINGS:
        return list(a.strings)
    raise ValueError(f"attribute '{a.name}': type {a.type} unsupported")


def make_attribute(name: str, value: Any):
    a = AttributeProto(name=name)
    if isinstance(value, bool) or isinstance(value, (int, np.integer)):
        a.type, a.i = A_INT, int(value)
    elif isinstance(value, (float, np.floating)):
        a.type, a.f = A_FLOAT, float(value)
    elif isinstance(value, str):
        a.type, a.s = A_STRING, value.encode()
    elif isinstance(value, bytes):
        a.type, a.s = A_STRING, value
    elif isinstance(value, np.ndarray):
        a.type = A_TENSOR
        a.t.CopyFrom(numpy_to_tensor("", value))
    elif isinstance(value, (list, tuple)):
        if all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) for v in value):
            a.type = A_INTS
            a.ints.extend(int(v) for v in value)
        elif all(isinstance(v, (int, float, np.number)) for v in value):
            a.type = A_FLOATS
            a.floats.extend(float(v) for v in value)
        elif all(isinstance(v, (str, bytes)) for v in value):
            a.type = A_STRINGS
            a.strings.extend(v.encode() if isinstance(v, str) else v for v in value)
        else:
            raise ValueError(f"attribute '{name}': mixed list")
    else:
        raise ValueError(f"attribute '{name}': {type(value).__name__} unsupported")
    return a


# ------------------------------------------------------------------ files
def load_model(path: str):
    m = ModelProto()
    with open(path, "rb") as f:
        m.ParseFromString(f.read())
    if not m.HasField("graph"):
        raise ValueError(f"{path}: ModelProto has no graph")
    return m


def save_model(model, path: str) -> None:
    with open(path, "wb") as f:
        f.write(model.SerializeToString())


def _dims_of(vi) -> Tuple[ONNSType, List[Any]]:
    t = vi.type.tensor_type
    shape: List[Any] = []
    for d in t.shape.dim:
        if d.dim_param:
            shape.append(d.dim_param)
        elif d.HasField("dim_value"):
            shape.append(int(d.dim_value))
        else:
            shape.append(None)
    return ONNSType.from_onnx(t.elem_type), shape


def import_onnx(model_path: str) -> Graph:
    """`.onnx` file -> Graph (c31/import_onnx.py:60-200 semantics)."""
    model = load_model(model_path)
    gp = model.graph
    graph = Graph()
    graph.name = gp.name or ""
    graph.opsets = {o.domain or "ai.onnx": int(o.version) for o in model.opset_import}
    init_names = {t.name for t in gp.initializer}
    for t in gp.initializer:
        tensor = graph.register_tensor(name=t.name, dtype=ONNSType.from_onnx(t.data_type),
                                       shape=[int(d) for d in t.dims], is_initializer=True)
        graph.initializers[t.name] = tensor
        graph.tensor_producer[t.name] = "INITIALIZER"
    for vi in gp.input:
        if vi.name in init_names:
            continue
        dtype, shape = _dims_of(vi)
        graph.inputs.append(graph.register_tensor(name=vi.name, dtype=dtype, shape=shape, is_initializer=False))
        graph.tensor_producer[vi.name] = "INPUT"
    for vi in gp.output:
        dtype, shape = _dims_of(vi)
        graph.outputs.append(graph.register_tensor(name=vi.name, dtype=dtype, shape=shape, is_initializer=False))
    for vi in gp.value_info:
        dtype, shape = _dims_of(vi)
        graph.register_tensor(vi.name, dtype=dtype, shape=shape)
    used = set()
    for idx, np_ in enumerate(gp.node):
        nid = generate_node_id(np_.name, np_.op_type, idx)
        if nid in used:
            base, k = nid, 1
            while f"{base}_{k}" in used:
                k += 1
            nid = f"{base}_{k}"
        used.add(nid)
        attrs = {a.name: _json_safe(attribute_value(a)) for a in np_.attribute}
        node = Node(id=nid, name=np_.name or "", op_type=np_.op_type, inputs=list(np_.input),
                    outputs=list(np_.output), attributes=attrs, domain=np_.domain or "")
        graph.add_node(node)
        for out in node.outputs:
            if out:
                graph.register_tensor(name=out)
                graph.set_producer(out, nid)
        if np_.op_type == "Constant":
            for a in np_.attribute:
                if a.name == "value" and (a.type == A_TENSOR or a.HasField("t")):
                    for out in node.outputs:
                        if out:
                            graph.register_tensor(name=out, dtype=ONNSType.from_onnx(a.t.data_type),
                                                  shape=[int(d) for d in a.t.dims], is_constant=True)
                    break
    for node in graph.nodes.values():  # inputs nobody declares still become tensors; validate() names them
        for name in node.inputs:
            if name and name not in graph.tensors:
                graph.register_tensor(name=name)
    graph.validate()  # structural checks + topological order
    weights, constants = read_initializers_and_constants(model)
    infer_shapes(graph, {**weights, **constants})
    return graph


def read_initializers_and_constants(source) -> Tuple[Dict[str, np.ndarray], Dict[str, np.ndarray]]:
    """(initializers, Constant-node outputs) as host arrays (c35/executor.py:23-88)."""
    model = load_model(source) if isinstance(source, str) else source
    weights = {t.name: tensor_to_numpy(t) for t in model.graph.initializer}
    constants: Dict[str, np.ndarray] = {}
    for n in model.graph.node:
        if n.op_type != "Constant":
            continue
        vals = [a for a in n.attribute if a.name in ("value", "value_float", "value_floats", "value_int",
                                                      "value_ints")]
        if len(vals) != 1:
            raise ValueError(f"Constant node '{n.name}' needs exactly one supported value attribute")
        a = vals[0]
        if a.name == "value":
            value = tensor_to_numpy(a.t)
        elif a.name == "value_float":
            value = np.array(a.f, np.float32)
        elif a.name == "value_floats":
            value = np.array(list(a.floats), np.float32)
        elif a.name == "value_int":
            value = np.array(a.i, np.int64)
        else:
            value = np.array(list(a.ints), np.int64)
        for out in n.output:
            if out:
                constants[out] = value
    return weights, constants


# ------------------------------------------------------------------ shape inference
def _bcast(*shapes):
    nd = max(len(s) for s in shapes)
    out = []
    for i in range(nd):
        dims = [s[i - nd + len(s)] for s in shapes if i - nd + len(s) >= 0]
        known = [d for d in dims if isinstance(d, int) and d != 1]
        if known:
            out.append(known[0])
        elif any(isinstance(d, str) for d in dims):
            out.append(next(d for d in dims if isinstance(d, str)))
        else:
            out.append(1)
    return out


def _conv_out(x, ks, attrs):
    s = attrs.get("strides", [1] * len(ks))
    d = attrs.get("dilations", [1] * len(ks))
    p = attrs.get("pads", [0] * (2 * len(ks)))
    out = []
    for i, k in enumerate(ks):
        n = x[2 + i]
        if not isinstance(n, int):
            out.append(None)
            continue
        out.append((n + p[i] + p[i + len(ks)] - d[i] * (k - 1) - 1) // s[i] + 1)
    return out


def _symbolic(x: Sequence[Any], fn) -> Optional[List[Any]]:
    """Apply a concrete shape function `fn` to a shape with one symbolic dim.

    The symbol is bound to two different probe sizes; output dims that do not
    move are concrete, dims that equal the probe are the symbol, anything else
    (a product such as batch*8) is left unknown (None)."""
    syms = {str(d) for d in x if not isinstance(d, int)}
    if not syms:
        return list(fn([int(d) for d in x]))
    if len(syms) != 1:
        return None
    sym = next(d for d in x if not isinstance(d, int))
    probes = (1009, 2003)
    outs = [list(fn([p if not isinstance(d, int) else d for d in x])) for p in probes]
    res: List[Any] = []
    for a, b in zip(*outs):
        res.append(a if a == b else sym if (a, b) == probes else None)
    return res


def infer_shapes(graph: Graph, values: Dict[str, np.ndarray]) -> None:
    """Fill missing tensor shapes/dtypes for the C3 op subset (symbolic batch kept)."""
    def shape(name):
        t = graph.tensors.get(name)
        if name in values:
            return list(np.asarray(values[name]).shape)
        return list(t.shape) if t is not None and t.shape else None

    def dtype(name):
        t = graph.tensors.get(name)
        return t.dtype if t is not None else ONNSType.FLOAT

    for nid in graph.node_order:
        n = graph.nodes[nid]
        out = [o for o in n.outputs if o]
        if all(shape(o) and all(isinstance(d, int) for d in shape(o)) for o in out):
            continue
        ins = [shape(i) if i else None for i in n.inputs]
        op, at = n.op_type, n.attributes
        res: Optional[List[List[Any]]] = None
        odt = dtype(n.inputs[0]) if n.inputs and n.inputs[0] else ONNSType.FLOAT
        try:
            if op in ("Relu", "Erf", "Sqrt", "Exp", "Reciprocal", "Softmax", "LayerNormalization",
                      "BatchNormalization", "Dropout", "Identity", "Cast"):
                res = [ins[0]]
            elif op in ("Add", "Sub", "Mul", "Div", "Pow", "Max", "Min"):
                res = [_bcast(*[s for s in ins if s is not None])]
            elif op == "Gemm":
                a, b = ins[0], ins[1]
                mdim = a[1] if at.get("transA", 0) else a[0]
                ndim = b[0] if at.get("transB", 0) else b[1]
                res = [[mdim, ndim]]
            elif op in ("MatMul", "QLinearMatMul"):
                a, b = ins[0], ins[3] if op == "QLinearMatMul" else ins[1]
                lead = _bcast(a[:-2], b[:-2]) if len(a) > 2 and len(b) > 2 else (a[:-2] if len(a) > 2 else b[:-2])
                res = [list(lead) + [a[-2], b[-1]]] if len(a) >= 2 else [[b[-1]]]
                if op == "QLinearMatMul":
                    odt = ONNSType.INT8
            elif op == "Conv":
                x, w = ins[0], ins[1]
                res = [[x[0], w[0]] + _conv_out(x, list(w[2:]), at)]
            elif op == "MaxPool":
                x = ins[0]
                res = [[x[0], x[1]] + _conv_out(x, list(at["kernel_shape"]), at)]
            elif op == "GlobalAveragePool":
                res = [ins[0][:2] + [1] * (len(ins[0]) - 2)]
            elif op == "Flatten":
                x = ins[0]
                ax = int(at.get("axis", 1)) % len(x)
                res = [_symbolic(x, lambda c: [math.prod(c[:ax]), math.prod(c[ax:])])]
            elif op == "Reshape":
                from .c35.engine import resolve_reshape_shape
                target = [int(v) for v in np.asarray(values[n.inputs[1]]).reshape(-1)]
                allowzero = int(at.get("allowzero", 0))
                res = [_symbolic(ins[0], lambda c: resolve_reshape_shape(c, target, allowzero))]
            elif op == "Transpose":
                x = ins[0]
                perm = at.get("perm") or list(range(len(x) - 1, -1, -1))
                res = [[x[p] for p in perm]]
            elif op == "Split":
                x = ins[0]
                ax = int(at.get("axis", 0)) % len(x)
                sizes = at.get("split") or (list(np.asarray(values[n.inputs[1]]).reshape(-1))
                                            if len(n.inputs) > 1 and n.inputs[1] in values else None)
                if not sizes:
                    sizes = [x[ax] // len(out)] * len(out)
                res = [x[:ax] + [int(sz)] + x[ax + 1:] for sz in sizes]
            elif op == "Gather":
                data, idx = ins[0], ins[1]
                ax = int(at.get("axis", 0)) % len(data)
                res = [data[:ax] + idx + data[ax + 1:]]
            elif op == "QuantizeLinear":
                res, odt = [ins[0]], ONNSType.INT8
            elif op == "DequantizeLinear":
                res, odt = [ins[0]], ONNSType.FLOAT
            elif op == "ArgMax":
                x = ins[0]
                ax = int(at.get("axis", 0)) % len(x)
                res = [x[:ax] + ([1] if int(at.get("keepdims", 1)) else []) + x[ax + 1:]]
                odt = ONNSType.INT64
            elif op in ("ReduceMean", "ReduceSum", "ReduceMax"):
                x = ins[0]
                axes = at.get("axes") or list(range(len(x)))
                axes = [a % len(x) for a in axes]
                keep = int(at.get("keepdims", 1))
                res = [[1 if i in axes else d for i, d in enumerate(x)] if keep else
                       [d for i, d in enumerate(x) if i not in axes]]
        except (TypeError, IndexError, KeyError):
            res = None
        if res is None or any(r is None for r in res):
            continue
        for o, sh in zip(out, res):
            t = graph.tensors.get(o)
            if t is None or not t.shape:
                graph.register_tensor(o, dtype=odt, shape=list(sh))
                continue
            if len(t.shape) == len(sh):  # merge: an inferred size replaces a declared symbol
                merged = []
                for d, e in zip(t.shape, sh):
                    if isinstance(d, int) and isinstance(e, int) and d != e:
                        raise ValueError(f"tensor '{o}': declared shape {t.shape} conflicts with inferred {sh}")
                    merged.append(e if isinstance(e, int) else d)
                t.shape = merged
            if t.dtype in (None, ONNSType.UNDEFINED):
                t.dtype = odt


# ------------------------------------------------------------------ writer
def export_model(graph: Graph, weights: Dict[str, np.ndarray], path: Optional[str] = None, opset: int = 17,
                 value_info: bool = True):
    """Graph + initializer arrays -> ModelProto (written to `path` when given).

    `value_info=False` leaves intermediate shapes out, as files from most
    exporters do; `import_onnx` then recovers them with `infer_shapes`."""
    m = ModelProto(ir_version=8, producer_name="hackathon_amd", producer_version="1")
    m.opset_import.add(domain="", version=opset)
    g = m.graph
    g.name = graph.name or "c3"

    def add_value_info(target, name):
        t = graph.tensors.get(name)
        vi = target.add(name=name)
        tt = vi.type.tensor_type
        tt.elem_type = t.dtype.to_onnx() if t is not None and t.dtype is not None else 1
        for d in (t.shape if t is not None and t.shape else []):
            dim = tt.shape.dim.add()
            if isinstance(d, (int, np.integer)):
                dim.dim_value = int(d)
            elif d is not None:
                dim.dim_param = str(d)
        return vi

    for t in graph.inputs:
        add_value_info(g.input, t.name)
    for t in graph.outputs:
        add_value_info(g.output, t.name)
    for name in graph.initializers:
        if name in weights:
            g.initializer.append(numpy_to_tensor(name, np.asarray(weights[name])))
    if not graph.node_order:
        graph.topological_sort()
    produced = set()
    for nid in graph.node_order:
        n = graph.nodes[nid]
        np_ = g.node.add(name=n.name or n.id, op_type=n.op_type, domain=n.domain or "")
        np_.input.extend(n.inputs)
        np_.output.extend(n.outputs)
        for k, v in (n.attributes or {}).items():
            if k.startswith("_"):
                continue
            np_.attribute.append(make_attribute(k, v))
        produced.update(o for o in n.outputs if o)
    outputs = {t.name for t in graph.outputs}
    for name in sorted(produced - outputs) if value_info else []:
        t = graph.tensors.get(name)
        if t is not None and t.shape:
            add_value_info(g.value_info, name)
    if path is not None:
        save_model(m, path)
    return m
