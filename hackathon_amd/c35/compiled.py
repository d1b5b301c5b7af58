"""Compiled execution of a C3.4 plan: launch groups, views, one slab, hipGraph.

The strict interpreter (executor.PlannedGraphExecutor) runs every kernel step
of a plan as its own registry launch with fp32 arena views, like the
reference.  `CompiledPlan` consumes the same plan and graph and lowers it for
the MI355X instead:

* Launch grouping: the steps of one node (c32 decompositions, e.g.
  im2col -> contract -> reshape -> bias for a Conv) become one launch, and a
  node's single-consumer epilogue neighbours fold into it: Relu and the
  residual Add+Relu chain into the conv/GEMM epilogue, a GELU FusedEWChain
  into the FFN GEMM epilogue, a residual Add into the output-projection
  GEMM, FusedAttentionScores + its P.V MatMul into one flash-attention launch
  writing straight into the FusedTransposeReshape layout, and
  QLinearMatMul -> DequantizeLinear -> bias (-> GELU) into one int8 GEMM.
  Under the "fp8" policy a GEMM the plan marks fp8 becomes a row-wise E4M3
  quantization of its activation plus one E4M3 GEMM (weights quantized per
  output channel once at compile time) with the same absorbed epilogue.
  Under the "fp4" policy a GEMM the plan marks fp4 becomes one W4A16 GEMM on
  its fp16 activation (weights quantized to MXFP4 once at compile time).
* Views: Reshape / Flatten / Split / Transpose produce strided views (no
  copies, no host syncs: shape tensors are read at compile time); a consumer
  that needs dense data materializes once.
* Layout: convolutional activations are channels-last (NHWC, channels
  padded to a vector multiple) between convolutions; graph inputs are
  converted once, and channel-last data feeds GlobalAveragePool / MaxPool /
  elementwise chains directly.
* Precision: the plan's policy ("fp32" | "bf16" | "fp16" | "w8a8" | "fp8" | "fp4") picks the
  storage dtype of every activation and the MFMA input type of every
  contraction; weights are packed and converted once at compile time.
* Memory: activation buffers are re-planned over the grouped launch order
  with the C3.4 best-fit pool into one hipMalloc slab (views extend their
  base's lifetime).
* Replay: the launch list is a native c3h_op program, captured once into a
  hipGraph and replayed per batch (no Python per kernel).
"""

from __future__ import annotations

import ctypes as C
import os
import math
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import _lib
from ..c3common.ir.graph import Graph, Node
from ..c34.execution_plan import ExecutionPlan
from ..c34.memory_pool import DeviceMemoryPool
from ..device import BF16, Buffer, DeviceArray, PinnedArray, Stream, device_props, dtype_code, init, synchronize
from . import engine as E

_POLICY_ACT = {"fp32": np.dtype(np.float32), "bf16": BF16, "fp16": np.dtype(np.float16), "w8a8": BF16,
               "fp8": np.dtype(np.float16), "fp4": np.dtype(np.float16)}
_MM_CODE = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16, "w8a8": _lib.BF16, "fp8": _lib.F16,
            "fp4": _lib.F16}
# c3h_layernorm's vector path (the only one with an int8 output): 8-wide
# vectors, at most 8 per lane of one wave (memory_bound.hip: 512 * kLnVec).
LN_QUANT_MAX_COLS = 4096


def quant_scale_ok(scale: float) -> bool:
    """The C side's quant_scale_ok: the scale, as the fp32 the launch receives,
    is a positive normal number (2^-126 <= s <= FLT_MAX)."""
    with np.errstate(over="ignore"):
        s = np.float32(scale)
    return bool(np.isfinite(s) and s >= np.float32(2.0 ** -126))


_DTYPE_NAME = {np.dtype(np.float32): "fp32", np.dtype(np.float16): "fp16", BF16: "bf16", np.dtype(np.int8): "int8",
               np.dtype(np.int32): "int32", np.dtype(np.int64): "int64", np.dtype(np.uint8): "u8"}


# ---------------------------------------------------------------- values and buffers
class Buf:
    """A device allocation: slab-planned activation, persistent weight, or input."""

    __slots__ = ("nbytes", "kind", "array", "first", "last", "offset", "name")

    def __init__(self, nbytes: int, kind: str, array: Optional[DeviceArray] = None, name: str = "") -> None:
        self.nbytes = int(nbytes)
        self.kind = kind  # "slab" | "weight" | "input"
        self.array = array
        self.first = -1
        self.last = -1
        self.offset = 0
        self.name = name

    def touch(self, idx: int) -> None:
        if self.first < 0:
            self.first = idx
        self.last = max(self.last, idx)


@dataclass
class Val:
    """A graph value: logical (ONNX) shape over a storage buffer."""

    shape: Tuple[int, ...]
    dtype: np.dtype
    buf: Optional[Buf]
    offset: int = 0                                  # elements
    strides: Optional[Tuple[int, ...]] = None        # logical strides in elements (None: dense)
    layout: str = "dense"                            # "dense" | "nhwc"
    c_stride: int = 0                                # NHWC channel stride
    host: Optional[np.ndarray] = None                # host copy of small constants

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    def logical_strides(self) -> Tuple[int, ...]:
        if self.layout == "nhwc":
            n, c, h, w = self.shape
            cs = self.c_stride
            return (h * w * cs, 1, w * cs, cs)
        return self.strides if self.strides is not None else tuple(E.dense_strides(self.shape))

    @property
    def dense(self) -> bool:
        if self.layout != "dense":
            return False
        if self.strides is None:
            return True
        return all(n == 1 or s == d for n, s, d in zip(self.shape, self.strides, E.dense_strides(self.shape)))


@dataclass
class _Epi:
    """Epilogue state of one GEMM/conv launch (see c3h_epilogue)."""

    bias: Optional[Val] = None
    residual: Optional[Val] = None
    act: int = 0
    prog: List[Tuple[int, int, int, float]] = field(default_factory=list)
    imm: List[float] = field(default_factory=list)
    x_name: str = ""
    final: str = ""
    absorbed: List[str] = field(default_factory=list)
    row_max: Optional["Val"] = None    # block-maxima side output (c3h_epilogue.row_max)


def _numel_bytes(shape, dtype) -> int:
    return math.prod(shape) * np.dtype(dtype).itemsize


class _Launch:
    __slots__ = ("build", "stream")

    def __init__(self, build: Callable[[Callable[[Val], int]], Tuple[int, Any]], stream: int = 0) -> None:
        self.build = build
        self.stream = stream


class CompiledPlan:
    """A plan lowered to grouped launches over one slab (see module docstring)."""

    def __init__(self, graph: Graph, plan: ExecutionPlan, host_weights: Dict[str, Any],
                 host_constants: Optional[Dict[str, Any]] = None, policy: str = "fp32",
                 use_graph: bool = True, fuse_stem: bool = True, concurrent: bool = True,
                 keep_values: bool = False) -> None:
        init()
        if policy not in _POLICY_ACT:
            raise ValueError(f"unknown precision policy {policy!r}")
        issues = plan.validate()
        if issues:
            raise ValueError("C3.4 execution plan is invalid: " + "; ".join(issues[:10]))
        self.graph, self.plan, self.policy = graph, plan, policy
        self.act_dtype = _POLICY_ACT[policy]
        self.mm_code = _MM_CODE[policy]
        self.batch = plan.batch_size
        self.weights_src = dict(host_weights)
        self.weights_src.update(host_constants or {})
        self.vals: Dict[str, Val] = {}
        self.launches: List[_Launch] = []
        self.bufs: List[Buf] = []
        self.keep: List[Any] = []          # persistent device arrays / ctypes objects
        self.inputs: Dict[str, Val] = {}
        self.consumed: set = set()         # node ids already lowered into an earlier launch
        self.node_kinds: List[str] = []     # launch labels (for reporting)
        self._rounded: Dict[str, str] = {}  # values rounded to a storage type in registers only
        self.launch_meta: List[Dict[str, Any]] = []  # per launch: kind, algorithmic flops and bytes
        self.launch_rw: List[Tuple[List[Buf], List[Buf]]] = []  # per launch: buffers read, buffers written
        self.concurrent = concurrent and not os.environ.get("C3H_SERIAL_PLAN")
        self.pairs: List[int] = []         # launch p and p + 1 run concurrently (p + 1 on the side stream)
        self.use_graph = use_graph
        self.fuse_stem = fuse_stem
        # keep_values: every slab buffer gets memory of its own (no reuse), so
        # each value the program stores can be read back after a run
        self.keep_values = keep_values
        self._cus = int(device_props().compute_units)
        self._graph_exec = None
        self._stream = Stream()
        self._consumers = self._consumer_map()
        # per node: the contraction type the plan's precision profile chose
        self._node_compute = {k.node_id: (k.precision_profile or {}).get("compute_dtype")
                              for k in plan.kernel_steps}
        self._lower()
        synchronize()  # compile-time weight conversions (null stream) before the plan's stream runs
        self._finalize()

    # ---------------------------------------------------------------- analysis helpers
    def _consumer_map(self) -> Dict[str, List[str]]:
        cons: Dict[str, List[str]] = {}
        for nid in self._node_order():
            for i in self.graph.nodes[nid].inputs:
                if i:
                    cons.setdefault(i, []).append(nid)
        return cons

    def _node_order(self) -> List[str]:
        order, seen = [], set()
        for s in self.plan.kernel_steps:
            if s.node_id not in seen:
                seen.add(s.node_id)
                order.append(s.node_id)
        return order

    def _single_consumer(self, tensor: str) -> Optional[Node]:
        outs = {t.name for t in self.graph.outputs}
        cons = self._consumers.get(tensor, [])
        if tensor in outs or len(set(cons)) != 1:
            return None
        return self.graph.nodes[cons[0]]

    def _is_output(self, tensor: str) -> bool:
        return any(t.name == tensor for t in self.graph.outputs)

    def _out_dtype(self, tensor: str) -> np.dtype:
        return np.dtype(np.float32) if self._is_output(tensor) else self.act_dtype

    # ---------------------------------------------------------------- value helpers
    def _weight_host(self, name: str) -> np.ndarray:
        v = self.weights_src[name]
        return v.get() if isinstance(v, DeviceArray) else np.asarray(v)

    def _persist(self, arr: DeviceArray) -> Buf:
        self.keep.append(arr)
        return Buf(arr.nbytes, "weight", arr)

    def _weight_val(self, name: str, dtype=None) -> Val:
        """A weight as a device value (converted to `dtype` if given)."""
        key = (name, None if dtype is None else np.dtype(dtype).str if np.dtype(dtype) != BF16 else "bf16")
        cache = self.__dict__.setdefault("_wcache", {})
        if key in cache:
            return cache[key]
        src = self.weights_src[name]
        if isinstance(src, DeviceArray):
            arr = src
        else:
            arr = DeviceArray.from_host(np.ascontiguousarray(np.asarray(src)))
        if dtype is not None and np.dtype(dtype) != arr.dtype:
            out = DeviceArray.empty(arr.shape, dtype)
            E.cast_into(arr, out)
            arr = out
        self._note_weight_store(name, arr.dtype)
        host = np.asarray(src) if not isinstance(src, DeviceArray) and np.asarray(src).size <= 4096 else None
        v = Val(tuple(arr.shape), arr.dtype, self._persist(arr), host=host)
        cache[key] = v
        return v

    def _note_weight_store(self, name: str, dtype) -> None:
        """Remember the narrowest type a weight is stored in on the device."""
        store = self.__dict__.setdefault("_weight_store", {})
        if np.dtype(dtype).itemsize == 2 or name not in store:
            store[name] = np.dtype(dtype)

    def _host_value(self, name: str) -> Optional[np.ndarray]:
        if name in self.weights_src:
            return self._weight_host(name)
        v = self.vals.get(name)
        return None if v is None else v.host

    def _new(self, shape, dtype, layout="dense", c_stride=0) -> Val:
        shape = tuple(int(d) for d in shape)
        if layout == "nhwc":
            n, c, h, w = shape
            nbytes = n * h * w * c_stride * np.dtype(dtype).itemsize
        else:
            nbytes = _numel_bytes(shape, dtype)
        b = Buf(max(nbytes, 1), "slab")
        self.bufs.append(b)
        return Val(shape, np.dtype(dtype), b, layout=layout, c_stride=c_stride)

    def _get(self, name: str) -> Val:
        if name in self.vals:
            return self.vals[name]
        if name in self.weights_src:
            v = self._weight_val(name)
            self.vals[name] = v
            return v
        raise KeyError(f"compiled plan: value '{name}' is not available")

    def _emit(self, kind: str, build, reads: Sequence[Val] = (), writes: Sequence[Val] = (),
              flops: float = 0.0, skip_bytes: Sequence[Val] = (), extra_bytes: int = 0, info: str = "") -> None:
        """Append one launch; records buffer lifetimes and algorithmic work.

        `bytes` is the launch's algorithmic HBM traffic: every operand read
        once and every output written once (logical sizes, no padding).  A
        read the launch touches only partly (a gathered table) is named in
        `skip_bytes` and its touched bytes given as `extra_bytes`.  `info`
        describes the launch's shape for per-launch reports.
        """
        idx = len(self.launches)
        seen = set()
        nbytes = 0
        for v in list(reads) + list(writes):
            if v is None:
                continue
            if v.buf is not None:
                v.buf.touch(idx)
            key = (id(v.buf), v.offset, v.shape, v.strides)
            if key not in seen:
                seen.add(key)
                if not any(v is sv for sv in skip_bytes):
                    nbytes += v.size * v.dtype.itemsize
        nbytes += int(extra_bytes)
        self.launches.append(_Launch(build))
        self.launch_rw.append(([v.buf for v in reads if v is not None and v.buf is not None],
                               [v.buf for v in writes if v is not None and v.buf is not None]))
        self.node_kinds.append(kind)
        self.launch_meta.append({"kind": kind, "flops": float(flops), "bytes": int(nbytes),
                                 "node": getattr(self, "_cur_node", None), "info": info})

    def _ptr(self, v: Val, resolve) -> int:
        return resolve(v.buf) + v.offset * v.dtype.itemsize

    def _dense(self, v: Val, dtype=None) -> Val:
        """`v` as a dense row-major value (materialized once if strided/NHWC/other dtype)."""
        dtype = v.dtype if dtype is None else np.dtype(dtype)
        if v.dense and dtype == v.dtype:
            return v
        out = self._new(v.shape, dtype)
        src = v
        if dtype != v.dtype and not v.dense:
            tmp = self._new(v.shape, v.dtype)
            self._copy_strided(v, tmp)
            src = tmp
        if src.dense:
            self._cast(src, out)
        else:
            self._copy_strided(src, out)
        return out

    def _copy_strided(self, src: Val, dst: Val) -> None:
        strides = src.logical_strides()
        shape = src.shape

        def build(r, src=src, dst=dst, shape=shape, strides=strides):
            a = _lib.CopyArgs()
            a.in_, a.out, a.elem_bytes, a.rank = self._ptr(src, r), self._ptr(dst, r), src.dtype.itemsize, len(shape)
            for d, (n, s) in enumerate(zip(shape, strides)):
                a.shape[d], a.in_stride[d] = n, s
            a.in_offset = 0
            return a
        self._emit("copy", build, [src], [dst])

    def _cast(self, src: Val, dst: Val) -> None:
        def build(r, src=src, dst=dst):
            a = _lib.CastArgs()
            a.in_, a.out, a.count = self._ptr(src, r), self._ptr(dst, r), src.size
            a.in_dtype, a.out_dtype = dtype_code(src.dtype), dtype_code(dst.dtype)
            return a
        self._emit("cast", build, [src], [dst])

    # ---------------------------------------------------------------- lowering driver
    def _lower(self) -> None:
        for t in self.graph.inputs:
            gt = self.graph.tensors[t.name]
            shape = tuple(self.batch if not isinstance(d, int) else int(d) for d in
                          [self._dim(d) for d in gt.shape])
            dtype = {"FLOAT": np.float32, "INT64": np.int64, "FLOAT16": np.float16, "INT32": np.int32}.get(
                gt.dtype.value, np.float32)
            buf = Buf(_numel_bytes(shape, dtype), "input", name=t.name)
            arr = DeviceArray.empty(shape, dtype)
            buf.array = self._keep(arr)
            v = Val(shape, np.dtype(dtype), buf)
            self.vals[t.name] = v
            self.inputs[t.name] = v
        for nid in self._node_order():
            if nid in self.consumed:
                continue
            node = self.graph.nodes[nid]
            handler = getattr(self, f"_op_{node.op_type}", None)
            if handler is None:
                raise NotImplementedError(f"compiled engine has no lowering for {node.op_type} (node {nid})")
            self._cur_node = nid
            handler(node)
        self._cur_node = None
        self.outputs: Dict[str, Val] = {}
        for t in self.graph.outputs:
            v = self.vals[t.name]
            if v.dtype.kind in "iu":  # integer outputs (ArgMax) keep their type
                v = v if v.dense else self._dense(v)
            elif v.dtype != np.float32 or not v.dense:
                v = self._dense(v, np.float32)
            self.outputs[t.name] = v
        end = len(self.launches)
        for v in self.outputs.values():
            v.buf.touch(end)

    def _keep(self, arr):
        self.keep.append(arr)
        return arr

    def _dim(self, d):
        try:
            v = int(d)
            return self.batch if v == -1 else v
        except (TypeError, ValueError):
            return self.batch

    def _shape_of(self, name: str) -> Tuple[int, ...]:
        t = self.graph.tensors.get(name)
        return tuple(self._dim(d) for d in t.shape) if t is not None and t.shape else ()

    # ---------------------------------------------------------------- finalize / run
    def _pair_independent_convs(self) -> None:
        """Let consecutive convolutions that do not depend on each other run
        concurrently: a residual block's downsample 1x1 conv and its first 3x3
        conv both read only the block input.  Independent means neither
        launch writes a buffer the other reads or writes (views count as
        their whole buffer).  Both launches' buffers get their slab lifetimes
        widened over the pair, so the best-fit pool cannot give one launch's
        output the memory of a buffer the other is still reading."""
        if not self.concurrent:
            return
        n, p = len(self.launches), 0
        while p + 1 < n:
            kinds = (self.node_kinds[p].split(":")[0], self.node_kinds[p + 1].split(":")[0])
            (r0, w0), (r1, w1) = self.launch_rw[p], self.launch_rw[p + 1]
            ids_w0, ids_w1 = {id(b) for b in w0}, {id(b) for b in w1}
            independent = not (ids_w0 & ({id(b) for b in r1} | ids_w1)) and not (ids_w1 & {id(b) for b in r0})
            if kinds == ("conv", "conv") and independent:
                self.pairs.append(p)
                for b in r0 + w0 + r1 + w1:
                    if b.first in (p, p + 1):
                        b.first = p
                    if b.last in (p, p + 1):
                        b.last = p + 1
                p += 2
            else:
                p += 1

    def _finalize(self) -> None:
        self._pair_independent_convs()
        pool = DeviceMemoryPool(alignment=256)
        slab_bufs = [b for b in self.bufs if b.kind == "slab" and b.first >= 0]
        by_first: Dict[int, List[Buf]] = {}
        by_last: Dict[int, List[Buf]] = {}
        for b in slab_bufs:
            by_first.setdefault(b.first, []).append(b)
            by_last.setdefault(b.last, []).append(b)
        slots: Dict[int, int] = {}
        for i in range(len(self.launches) + 1):
            for b in by_first.get(i, []):
                s = pool.alloc(b.nbytes, 256)
                slots[id(b)] = s
                b.offset = pool.describe(s)[0]
            for b in by_last.get(i, []):
                if i < len(self.launches) and not self.keep_values:
                    pool.free(slots[id(b)])
        self.slab_bytes = max(pool.stats().peak_reserved_bytes, 256)
        self.slab = Buffer(self.slab_bytes)
        base = self.slab.ptr

        def resolve(b: Buf) -> int:
            if b.kind == "slab":
                return base + b.offset
            return b.array.ptr

        self._args = []
        ops = (_lib.Op * len(self.launches))()  # one per launch, stream 0 (subset timing uses these)
        for i, launch in enumerate(self.launches):
            args = launch.build(resolve)
            self._args.append(args)
            ops[i].kind = _lib.OP_KIND[type(args)]
            ops[i].stream = 0
            ops[i].event = 0
            ops[i].args = C.cast(C.pointer(args), C.c_void_p)
        self._ops = ops
        self._streams = (C.c_void_p * 1)(self._stream.handle)
        # The program: launches in order; each pair (p, p + 1) forks p + 1 onto
        # the side stream after everything before p and joins it before p + 2.
        firsts = set(self.pairs)
        seq: List[Tuple[int, int, int, int]] = []  # (kind, stream, event, launch index or -1)
        ev = 0
        for i in range(len(self.launches)):
            if i - 1 in firsts:
                continue
            if i in firsts:
                seq += [(_lib.OP_EVENT_RECORD, 0, ev, -1), (_lib.OP_EVENT_WAIT, 1, ev, -1),
                        (ops[i].kind, 0, 0, i), (ops[i + 1].kind, 1, 0, i + 1),
                        (_lib.OP_EVENT_RECORD, 1, ev + 1, -1), (_lib.OP_EVENT_WAIT, 0, ev + 1, -1)]
                ev += 2
            else:
                seq.append((ops[i].kind, 0, 0, i))
        prog = (_lib.Op * len(seq))()
        for j, (kind, stream, event, li) in enumerate(seq):
            if li >= 0:
                C.memmove(C.byref(prog[j]), C.byref(ops[li]), C.sizeof(_lib.Op))
            prog[j].kind, prog[j].stream, prog[j].event = kind, stream, event
        self._prog, self._n_prog = prog, len(seq)
        if self.pairs:
            from ..device import Event, Stream as _Stream

            self._side = _Stream()
            self._events = [Event(timing=False) for _ in range(ev)]
            self._prog_streams = (C.c_void_p * 2)(self._stream.handle, self._side.handle)
            self._prog_events = (C.c_void_p * ev)(*[e.handle for e in self._events])
        else:
            self._prog_streams, self._prog_events = self._streams, None
        self._resolve = resolve
        self.output_arrays = {name: DeviceArray(resolve(v.buf) + v.offset * v.dtype.itemsize, v.shape, v.dtype,
                                                self.slab) for name, v in self.outputs.items()}
        if self.use_graph and self.launches:
            g = C.c_void_p()
            _lib.check(_lib.lib().c3h_program_capture(self._prog, self._n_prog, self._prog_streams,
                                                      len(self._prog_streams), self._prog_events,
                                                      len(self._events) if self.pairs else 0, C.byref(g)),
                       "c3h_program_capture")
            self._graph_exec = g.value

    @property
    def num_launches(self) -> int:
        return len(self.launches)

    def stored_dtypes(self) -> Dict[str, str]:
        """Storage type ("fp32", "bf16", "fp16", "int8", ...) of every graph
        tensor this program holds in memory.  Node outputs absent from the map
        never leave a fused launch: they exist only as fp32 values in
        registers (an absorbed bias, residual, activation or GELU step)."""
        return {k: _DTYPE_NAME.get(v.dtype, str(v.dtype)) for k, v in self.vals.items()
                if k not in self.weights_src and k not in self.inputs}

    def rounding_map(self) -> Dict[str, str]:
        """Every point where this program rounds a value to a storage type:
        weights as its launches read them, stored values, and values rounded
        in registers only (a LayerNorm output rounded to the activation type
        inside the launch that quantizes it).  What an emulation needs to
        round exactly where the program does."""
        return {**self.weight_dtypes(), **self.stored_dtypes(), **self._rounded}

    def rounded_in_registers(self) -> Dict[str, str]:
        """Values rounded to a storage type inside a launch and never stored."""
        return dict(self._rounded)

    def weight_dtypes(self) -> Dict[str, str]:
        """Storage type of every weight as the program's launches read it
        (e.g. "bf16" for a table or contraction weight converted at compile
        time; the narrowest when a weight has several device copies)."""
        return {k: _DTYPE_NAME.get(d, str(d)) for k, d in self.__dict__.get("_weight_store", {}).items()}

    def stage_inputs(self, feed: Dict[str, Any]) -> None:
        """Copy the batch into the input buffers on the compiled stream."""
        for name, v in self.inputs.items():
            src = feed[name]
            dst = v.buf.array
            if isinstance(src, DeviceArray):
                if src.nbytes != dst.nbytes:
                    raise ValueError(f"input '{name}' has {src.nbytes} bytes, plan expects {dst.nbytes}")
                _lib.check(_lib.lib().c3h_memcpy_d2d_async(dst.ptr, src.ptr, src.nbytes, self._stream.handle), "d2d")
            elif isinstance(src, tuple) and len(src) == 2 and isinstance(src[0], PinnedArray):
                # (pinned buffer, byte count): asynchronous on the compiled stream
                pinned, nbytes = src
                if nbytes != dst.nbytes:
                    raise ValueError(f"input '{name}' has {nbytes} bytes, plan expects {dst.nbytes}")
                _lib.check(_lib.lib().c3h_memcpy_h2d_async(dst.ptr, pinned.ptr, nbytes, self._stream.handle), "h2d")
            else:
                host = np.ascontiguousarray(np.asarray(src), dtype=dst.dtype)
                dst.copy_from_host(host, self._stream.handle)
                self._stream.synchronize()

    def launch(self) -> None:
        """Enqueue the whole program (hipGraph replay when captured)."""
        if self._graph_exec is not None:
            _lib.check(_lib.lib().c3h_graph_launch(self._graph_exec, self._stream.handle), "c3h_graph_launch")
        else:
            _lib.check(_lib.lib().c3h_program_run(self._prog, self._n_prog, self._prog_streams,
                                                  len(self._prog_streams), self._prog_events,
                                                  len(self._events) if self.pairs else 0), "c3h_program_run")

    def launches_of(self, kinds: Sequence[str]) -> List[int]:
        """Indices of launches whose kind (before any ':') is in `kinds`."""
        return [i for i, k in enumerate(self.node_kinds) if k.split(":")[0] in set(kinds)]

    def time_subset(self, indices: Sequence[int], reps: int = 20, repeat: int = 1) -> float:
        """Milliseconds per pass over the given launches, from a hipGraph
        holding only them (`repeat` passes back to back in one graph, so that
        a few-microsecond launch is not dominated by graph-launch overhead).

        The launches reuse the compiled buffers, so they see realistic data;
        the timing comes from HIP events recorded on the compiled stream
        around `reps` replays.  No launch reads a buffer it writes (the slab
        planner frees a launch's inputs only after placing its outputs), so
        repeating a launch recomputes the same result.
        """
        from ..device import Event

        idx = list(indices) * max(1, int(repeat))
        if not idx:
            return 0.0
        sub = (_lib.Op * len(idx))()
        for j, i in enumerate(idx):
            C.memmove(C.byref(sub[j]), C.byref(self._ops[i]), C.sizeof(_lib.Op))
        g = C.c_void_p()
        _lib.check(_lib.lib().c3h_program_capture(sub, len(idx), self._streams, 1, None, 0, C.byref(g)),
                   "c3h_program_capture")
        try:
            h = self._stream.handle
            _lib.check(_lib.lib().c3h_graph_launch(g.value, h), "c3h_graph_launch")
            start, end = Event(timing=True), Event(timing=True)
            start.record(self._stream)
            for _ in range(reps):
                _lib.check(_lib.lib().c3h_graph_launch(g.value, h), "c3h_graph_launch")
            end.record(self._stream)
            end.synchronize()
            return start.elapsed_ms(end) / reps / max(1, int(repeat))
        finally:
            _lib.lib().c3h_graph_destroy(g.value)

    def work(self, indices: Sequence[int]) -> Tuple[float, int]:
        """(algorithmic flops, algorithmic bytes) summed over the given launches."""
        return (sum(self.launch_meta[i]["flops"] for i in indices),
                sum(self.launch_meta[i]["bytes"] for i in indices))

    def run(self, feed: Dict[str, Any], sync: bool = True) -> Dict[str, DeviceArray]:
        self.stage_inputs(feed)
        self.launch()
        if sync:
            self._stream.synchronize()
            self.check_errors()
        return dict(self.output_arrays)

    @property
    def stream(self) -> Stream:
        return self._stream

    def __del__(self) -> None:
        g = getattr(self, "_graph_exec", None)
        if g and _lib._LIB is not None:
            _lib._LIB.c3h_graph_destroy(g)
            self._graph_exec = None

    # ================================================================ op lowerings
    # -- elementwise ------------------------------------------------------------------
    def _ew_val(self, inputs: List[Val], program, out_name: str, out_dtype=None) -> Val:
        """Elementwise program over `inputs`; NHWC inputs of one layout stay NHWC."""
        act = [v for v in inputs if v.size > 1]
        shape = E.broadcast_shape(*(v.shape for v in inputs))
        out_dtype = self._out_dtype(out_name) if out_dtype is None else out_dtype
        nhwc = [v for v in act if v.layout == "nhwc"]
        if nhwc and all(v.layout == "nhwc" and v.shape == shape and v.c_stride == nhwc[0].c_stride for v in act):
            cs = nhwc[0].c_stride
            phys = (shape[0], shape[2], shape[3], cs)
            out = self._new(shape, out_dtype, "nhwc", cs)
            pins = inputs
            strides_for = [tuple(E.dense_strides(phys)) if v.size > 1 else (0, 0, 0, 0) for v in inputs]
        else:
            pins = [v if v.size == 1 or v.layout == "dense" else self._dense(v) for v in inputs]
            out = self._new(shape, out_dtype)
            phys = shape
            strides_for = []
            for v in pins:
                ls = v.logical_strides()
                padded = (0,) * (len(shape) - len(v.shape)) + tuple(
                    0 if (d == 1 and shape[len(shape) - len(v.shape) + i] != 1) else s
                    for i, (d, s) in enumerate(zip(v.shape, ls)))
                strides_for.append(padded)

        def build(r, pins=pins, out=out, phys=phys, strides_for=strides_for, program=program):
            a = _lib.EwArgs()
            for j, v in enumerate(pins):
                a.in_[j] = self._ptr(v, r)
                a.in_dtype[j] = dtype_code(v.dtype)
                for d, s in enumerate(strides_for[j]):
                    a.stride[j][d] = s
            a.out, a.out_dtype, a.rank = self._ptr(out, r), dtype_code(out.dtype), len(phys)
            for d, s in enumerate(phys):
                a.shape[d] = s
            a.n_in, a.n_inst = len(pins), len(program)
            for i, (op, ra, rb, imm) in enumerate(program):
                a.inst[i].op, a.inst[i].a, a.inst[i].b, a.inst[i].imm = op, ra, rb, float(imm)
            return a
        self._emit("ew", build, pins, [out])
        return out

    def _op_Add(self, node):
        self._binary(node, _lib.EW_ADD)

    def _op_Sub(self, node):
        self._binary(node, _lib.EW_SUB)

    def _op_Mul(self, node):
        self._binary(node, _lib.EW_MUL)

    def _op_Div(self, node):
        self._binary(node, _lib.EW_DIV)

    def _binary(self, node, op):
        a, b = self._get(node.inputs[0]), self._get(node.inputs[1])
        self.vals[node.outputs[0]] = self._ew_val([a, b], [(op, 0, 1, 0.0)], node.outputs[0])

    def _unary(self, node, op):
        self.vals[node.outputs[0]] = self._ew_val([self._get(node.inputs[0])], [(op, 0, 0, 0.0)], node.outputs[0])

    def _op_Relu(self, node):
        self._unary(node, _lib.EW_RELU)

    def _op_Erf(self, node):
        self._unary(node, _lib.EW_ERF_AS)

    def _op_Sqrt(self, node):
        self._unary(node, _lib.EW_SQRT)

    def _op_Exp(self, node):
        self._unary(node, _lib.EW_EXP)

    def _op_FusedEWChain(self, node):
        ins = [self._get(i) for i in node.inputs]
        prog = E.compile_ew_program(node.attributes.get("_ops", []), len(ins))
        self.vals[node.outputs[0]] = self._ew_val(ins, prog, node.outputs[0])

    # -- metadata ops as views ---------------------------------------------------------------
    def _op_Constant(self, node):
        """Constant outputs arrive with the initializers (c35/executor.py:23-88) and load lazily."""
        for o in node.outputs:
            if o and o not in self.weights_src:
                raise KeyError(f"Constant node '{node.id}' output '{o}' not pre-loaded")

    def _view(self, v: Val, shape, strides, offset_delta=0) -> Val:
        return Val(tuple(shape), v.dtype, v.buf, v.offset + offset_delta, tuple(strides), "dense", 0, None)

    def _reshape_val(self, v: Val, shape: Tuple[int, ...]) -> Val:
        if v.layout == "nhwc":
            n, c, h, w = v.shape
            if h == 1 and w == 1 and v.c_stride == c:
                v = Val(v.shape, v.dtype, v.buf, v.offset, None)
            else:
                v = self._dense(v)
        strides = _reshape_strides(v.shape, v.logical_strides(), shape)
        if strides is None:
            v = self._dense(v)
            strides = tuple(E.dense_strides(shape))
        nv = self._view(v, shape, strides)
        if v.host is not None:
            nv.host = v.host.reshape(shape)
        return nv

    def _op_Reshape(self, node):
        x = self._get(node.inputs[0])
        target = self._host_value(node.inputs[1])
        if target is None:
            raise NotImplementedError("Reshape with a runtime shape tensor")
        shape = E.resolve_reshape_shape(x.shape, [int(v) for v in np.asarray(target).reshape(-1)],
                                        int(node.attributes.get("allowzero", 0)))
        self.vals[node.outputs[0]] = self._reshape_val(x, shape)

    def _op_Flatten(self, node):
        x = self._get(node.inputs[0])
        axis = int(node.attributes.get("axis", 1))
        axis = axis + len(x.shape) if axis < 0 else axis
        self.vals[node.outputs[0]] = self._reshape_val(x, (math.prod(x.shape[:axis]), math.prod(x.shape[axis:])))

    def _transpose_val(self, x: Val, perm) -> Val:
        if x.layout == "nhwc":
            x = self._dense(x)
        st = x.logical_strides()
        return self._view(x, [x.shape[p] for p in perm], [st[p] for p in perm])

    def _op_Transpose(self, node):
        x = self._get(node.inputs[0])
        perm = node.attributes.get("perm")
        perm = list(range(len(x.shape) - 1, -1, -1)) if perm is None else [int(p) for p in perm]
        self.vals[node.outputs[0]] = self._transpose_val(x, perm)

    def _op_FusedTransposeReshape(self, node):
        x = self._get(node.inputs[0])
        perm = [int(p) for p in node.attributes.get("perm")]
        t = self._transpose_val(x, perm)
        target = self._host_value(node.inputs[1])
        shape = E.resolve_reshape_shape(t.shape, [int(v) for v in np.asarray(target).reshape(-1)],
                                        int(node.attributes.get("allowzero", 0)))
        self.vals[node.outputs[0]] = self._reshape_val(t, shape)

    def _op_Split(self, node):
        x = self._get(node.inputs[0])
        if x.layout == "nhwc":
            x = self._dense(x)
        axis = int(node.attributes.get("axis", 0))
        axis = axis + len(x.shape) if axis < 0 else axis
        sizes = list(node.attributes.get("split", []) or [])
        if not sizes and len(node.inputs) > 1 and node.inputs[1]:
            sizes = [int(v) for v in np.asarray(self._host_value(node.inputs[1])).reshape(-1)]
        if not sizes:
            n = len([o for o in node.outputs if o])
            sizes = [x.shape[axis] // n] * n
        st = x.logical_strides()
        start = 0
        for name, size in zip(node.outputs, sizes):
            shape = list(x.shape)
            shape[axis] = size
            if name:
                self.vals[name] = self._view(x, shape, st, start * st[axis])
            start += size

    # -- GEMM family ------------------------------------------------------------------------
    def _packed_weight_nk(self, name: str, trans_b: int, dtype) -> Tuple[Val, int, int]:
        """Weight as B^T [n][k] (K-contiguous) in `dtype`, k padded to a multiple of 8."""
        cache = self.__dict__.setdefault("_pcache", {})
        key = (name, trans_b, str(np.dtype(dtype)) if np.dtype(dtype) != BF16 else "bf16")
        if key in cache:
            return cache[key]
        w = self._weight_host(name).astype(np.float32)
        if w.ndim != 2:
            raise ValueError(f"GEMM weight {name} must be rank 2")
        nk = w if trans_b else w.T
        n, k = nk.shape
        kp = (k + 7) // 8 * 8 if np.dtype(dtype).itemsize == 2 else k
        host = np.zeros((n, kp), np.float32)
        host[:, :k] = nk
        dev32 = DeviceArray.from_host(host)
        arr = dev32 if np.dtype(dtype) == np.float32 else DeviceArray.empty((n, kp), dtype)
        if arr is not dev32:
            E.cast_into(dev32, arr)
        v = Val((n, kp), np.dtype(dtype), self._persist(arr))
        self._note_weight_store(name, dtype)
        cache[key] = (v, n, k)
        return cache[key]

    def _bias_val(self, name: Optional[str]) -> Optional[Val]:
        if not name:
            return None
        return self._weight_val(name, np.float32)

    def _scalar_const(self, name: str) -> Optional[float]:
        h = self._host_value(name)
        if h is None or np.asarray(h).size != 1:
            return None
        return float(np.asarray(h).reshape(-1)[0])

    # -- epilogue absorption -------------------------------------------------------------------
    _PROG_CODES = {"Add": _lib.EW_ADD, "Sub": _lib.EW_SUB, "Mul": _lib.EW_MUL, "Div": _lib.EW_DIV,
                   "Relu": _lib.EW_RELU, "Erf": _lib.EW_ERF, "Sqrt": _lib.EW_SQRT, "Exp": _lib.EW_EXP}

    def _absorb_node(self, node: Node, cur: str, shape: Tuple[int, ...], st: "_Epi") -> Optional[str]:
        """Fold one consumer node of `cur` into the epilogue state; returns its output name.

        The epilogue applies bias -> residual -> act -> linear program in that
        order (c3hip.h), so a stage can only be taken while every later stage
        is still empty.  Program operands may be the value entering the
        program (x), the previous result, or scalar constants.
        """
        if node.op_type == "FusedEWChain":
            steps = []
            for e in node.attributes.get("_ops", []):
                ins = [node.inputs[r] if isinstance(r, int) else r for r in e.get("inputs", [])]
                steps.append((e["op"], ins, e.get("output", "")))
            if steps:
                steps[-1] = (steps[-1][0], steps[-1][1], node.outputs[0])
        elif node.op_type in self._PROG_CODES:
            steps = [(node.op_type, [i for i in node.inputs if i], node.outputs[0])]
        else:
            return None
        n = shape[-1]
        for op, ins, out in steps:
            if cur not in ins:
                return None
            others = [i for i in ins if i != cur]
            if op == "Add" and len(others) == 1 and not st.act and not st.prog:
                o = others[0]
                if st.bias is None and o in self.weights_src and self._weight_host(o).size == n and \
                        self._weight_host(o).shape[-1:] == (n,):
                    st.bias = self._weight_val(o, np.float32)
                    cur = out
                    continue
                v = self.vals.get(o)
                if st.residual is None and v is not None and v.shape == tuple(shape) and v.host is None:
                    st.residual = v
                    cur = out
                    continue
            if op == "Relu" and not st.act and not st.prog:
                st.act = 1
                cur = out
                continue
            if op not in self._PROG_CODES or len(st.prog) >= 16:
                return None
            if not st.prog:
                st.x_name = cur
            regs = []
            for i in ins:
                if i == cur:
                    regs.append(1)
                elif i == st.x_name:
                    regs.append(0)
                else:
                    s = self._scalar_const(i)
                    if s is None:
                        return None
                    if s in st.imm:
                        regs.append(2 + st.imm.index(s))
                    elif len(st.imm) < 8:
                        st.imm.append(s)
                        regs.append(1 + len(st.imm))
                    else:
                        return None
            if len(regs) == 1:
                regs = regs * 2
            if len(regs) != 2:
                return None
            st.prog.append((self._PROG_CODES[op], regs[0], regs[1], 0.0))
            cur = out
        return cur

    def _absorb_tail(self, out_name: str, shape: Tuple[int, ...], st: "_Epi") -> "_Epi":
        """Absorb the single-consumer elementwise successors of a GEMM/conv output."""
        import copy as _copy
        st.final = out_name
        while True:
            nxt = self._single_consumer(st.final)
            if nxt is None or nxt.id in self.consumed:
                break
            trial = _copy.copy(st)
            trial.prog, trial.imm = list(st.prog), list(st.imm)
            res = self._absorb_node(nxt, st.final, shape, trial)
            if res is None:
                break
            trial.final = res
            trial.absorbed = st.absorbed + [nxt.id]
            st = trial
        self.consumed.update(st.absorbed)
        _gelu_program_to_act(st)
        return st

    def _fill_epi(self, e, st: "_Epi", r, alpha: float = 1.0, beta: float = 1.0, bias_mode: Optional[int] = None):
        e.bias = self._ptr(st.bias, r) if st.bias is not None else None
        e.residual = self._ptr(st.residual, r) if st.residual is not None else None
        e.alpha, e.beta = alpha, beta
        e.bias_mode = (2 if st.bias is not None else 0) if bias_mode is None else bias_mode
        e.act = st.act
        e.n_imm, e.n_inst = len(st.imm), len(st.prog)
        for i, v in enumerate(st.imm):
            e.imm[i] = v
        for i, (op, ra, rb, iv) in enumerate(st.prog):
            e.inst[i].op, e.inst[i].a, e.inst[i].b, e.inst[i].imm = op, ra, rb, iv
        if st.row_max is not None:
            e.row_max, e.row_max_ld = self._ptr(st.row_max, r), st.row_max.shape[-1]

    def _note_row_max_site(self, st: "_Epi", out: Val, m: int, n: int, alpha: float = 1.0, beta: float = 1.0,
                            bias_mode: Optional[int] = None) -> None:
        """Remember the launch just emitted as able to write its rows' block
        maxima (c3h_epilogue.row_max): a GEMM whose epilogue the kernels keep
        in registers (alpha = beta = 1, no bias or a per-column one, at most
        ReLU, no program) into a dense float output with n % 4 == 0."""
        bm = (2 if st.bias is not None else 0) if bias_mode is None else bias_mode
        if st.prog or st.act > 1 or alpha != 1.0 or beta != 1.0 or bm not in (0, 2) or n % 4:
            return
        if out.dtype not in (np.dtype(np.float32), np.dtype(np.float16), BF16) or not out.dense or out.offset:
            return
        self.__dict__.setdefault("_row_max_sites", {})[st.final] = (len(self.launches) - 1, st, m, n, out)

    def _epi_reads(self, st: "_Epi") -> List[Val]:
        return [v for v in (st.bias, st.residual) if v is not None]

    def _finish_residual(self, st: "_Epi", out: Val) -> None:
        """Bring an absorbed residual into the output's storage dtype/layout."""
        res = st.residual
        if res is None:
            return
        if out.layout == "nhwc":
            if not (res.layout == "nhwc" and res.c_stride == out.c_stride and res.dtype == out.dtype):
                st.residual = self._nhwc_input(res, out.dtype, out.c_stride)
        elif res.dtype != out.dtype or not res.dense:
            st.residual = self._dense(res, out.dtype)

    def _fp8_weight(self, name: str, trans_b: int) -> Tuple[Val, Val, int, int]:
        """Weight as E4M3 codes B^T [n][k] + per-output-channel scales [n] (quantized on the GPU)."""
        cache = self.__dict__.setdefault("_f8cache", {})
        key = (name, trans_b)
        if key not in cache:
            w32, n, k = self._packed_weight_nk(name, trans_b, np.float32)
            codes = DeviceArray.empty((n, k), np.uint8)
            scales = DeviceArray.empty((n,), np.float32)
            q = _lib.Fp8QuantArgs()
            q.x, q.out, q.scale = w32.buf.array.ptr, codes.ptr, scales.ptr
            q.rows, q.cols, q.ldx, q.ldo, q.x_dtype = n, k, k, k, _lib.F32
            _lib.launch(q, None)
            cache[key] = (Val((n, k), np.dtype(np.uint8), self._persist(codes)),
                          Val((n,), np.dtype(np.float32), self._persist(scales)), n, k)
        return cache[key]

    def _fp4_weight(self, name: str, trans_b: int) -> Tuple[Val, Val, int, int]:
        """Weight as MXFP4: E2M1 codes of B^T [n][k/2] + E8M0 block exponents [n][k/32] (quantized on the GPU)."""
        cache = self.__dict__.setdefault("_f4cache", {})
        key = (name, trans_b)
        if key not in cache:
            w32, n, k = self._packed_weight_nk(name, trans_b, np.float32)
            if k % 32:
                raise NotImplementedError(f"MXFP4 weight {name}: K={k} is not a multiple of 32")
            codes = DeviceArray.empty((n, k // 2), np.uint8)
            scales = DeviceArray.empty((n, k // 32), np.uint8)
            q = _lib.Mxfp4QuantArgs()
            q.x, q.codes, q.scales = w32.buf.array.ptr, codes.ptr, scales.ptr
            q.rows, q.cols, q.ldx, q.ldc, q.lds, q.x_dtype = n, k, k, k // 2, k // 32, _lib.F32
            _lib.launch(q, None)
            cache[key] = (Val((n, k // 2), np.dtype(np.uint8), self._persist(codes)),
                          Val((n, k // 32), np.dtype(np.uint8), self._persist(scales)), n, k)
        return cache[key]

    def _gemm_w4a16(self, node, a: Val, w_name: str, trans_b: int, st: "_Epi", alpha: float, beta: float,
                    bmode, out_shape: Tuple[int, ...]) -> Val:
        """W4A16 GEMM of the fp16 activation with the MXFP4 weight and the epilogue `st`."""
        m, k = math.prod(a.shape[:-1]), a.shape[-1]
        wc, ws, n, kw = self._fp4_weight(w_name, trans_b)
        if kw != k:
            raise NotImplementedError(f"GEMM {node.id}: K={k} vs weight K={kw}")
        a2 = a if (a.dense and a.dtype == np.dtype(np.float16)) else self._dense(a, np.dtype(np.float16))
        out = self._new(out_shape, self._out_dtype(st.final))
        self._finish_residual(st, out)

        def build(r, a2=a2, out=out, st=st):
            g = _lib.W4A16GemmArgs()
            g.a, g.b_codes, g.b_scales, g.out = self._ptr(a2, r), self._ptr(wc, r), self._ptr(ws, r), self._ptr(out, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldbs, g.ldo = m, n, k, k, k // 2, k // 32, n
            g.out_dtype = dtype_code(out.dtype)
            self._fill_epi(g.epi, st, r, alpha, beta, bmode)
            return g
        self._emit(f"gemm_w4a16:{node.op_type}", build, [a2, wc, ws] + self._epi_reads(st), [out],
                   flops=2.0 * m * n * k)
        self._note_row_max_site(st, out, m, n, alpha, beta, bmode)
        return out

    def _gemm_fp8(self, node, a: Val, w_name: str, trans_b: int, st: "_Epi", alpha: float, beta: float,
                  bmode, out_shape: Tuple[int, ...]) -> Val:
        """Row-wise E4M3 quantization of A, then the E4M3 GEMM with the epilogue `st`."""
        m, k = math.prod(a.shape[:-1]), a.shape[-1]
        wq, ws, n, kw = self._fp8_weight(w_name, trans_b)
        if kw != k:
            raise NotImplementedError(f"GEMM {node.id}: K={k} vs weight K={kw}")
        a2 = a if (a.dense and a.dtype == self.act_dtype) else self._dense(a, self.act_dtype)
        qa = self._new((m, k), np.uint8)
        sa = self._new((m,), np.float32)
        xcode = dtype_code(a2.dtype)

        def qbuild(r, a2=a2, qa=qa, sa=sa):
            q = _lib.Fp8QuantArgs()
            q.x, q.out, q.scale = self._ptr(a2, r), self._ptr(qa, r), self._ptr(sa, r)
            q.rows, q.cols, q.ldx, q.ldo, q.x_dtype = m, k, k, k, xcode
            return q
        self._emit("quantize_fp8", qbuild, [a2], [qa, sa])
        out = self._new(out_shape, self._out_dtype(st.final))
        self._finish_residual(st, out)

        def build(r, out=out, st=st):
            g = _lib.Fp8GemmArgs()
            g.a, g.b, g.a_scale, g.b_scale = self._ptr(qa, r), self._ptr(wq, r), self._ptr(sa, r), self._ptr(ws, r)
            g.out = self._ptr(out, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.out_dtype = m, n, k, k, k, n, dtype_code(out.dtype)
            self._fill_epi(g.epi, st, r, alpha, beta, bmode)
            return g
        self._emit(f"gemm_fp8:{node.op_type}", build, [qa, sa, wq, ws] + self._epi_reads(st), [out],
                   flops=2.0 * m * n * k)
        self._note_row_max_site(st, out, m, n, alpha, beta, bmode)
        return out

    def _gemm_epi_state(self, node, bias_name: Optional[str], act: int, m: int, n: int,
                        out_shape: Tuple[int, ...]) -> Tuple["_Epi", Optional[int]]:
        """Bias mode + the epilogue state with single-consumer tails absorbed."""
        bmode = None
        st = _Epi(act=act)
        if bias_name:
            bias = self._bias_val(bias_name)
            bmode = 2 if bias.size == n else (1 if bias.size == 1 else 4 if bias.size == m * n else -1)
            if bmode < 0:
                raise NotImplementedError(f"GEMM {node.id}: bias of {bias.size} elements")
            st.bias = bias
        if not act and bmode in (None, 2):
            st = self._absorb_tail(node.outputs[0], out_shape, st)
        else:
            st.final = node.outputs[0]
        return st, bmode

    def _gemm_node(self, node, a: Val, w_name: str, trans_b: int, bias_name: Optional[str], alpha: float,
                   beta: float, act: int, lead: Tuple[int, ...]) -> None:
        """out[lead..., n] = epilogue(alpha * A @ W + beta * bias) with absorbed tails."""
        m, k = math.prod(a.shape[:-1]), a.shape[-1]
        low = self._node_compute.get(node.id)
        if low in ("fp8", "fp4"):
            if (low, self.policy) not in (("fp8", "fp8"), ("fp8", "fp4"), ("fp4", "fp4")):
                raise ValueError(f"GEMM {node.id}: plan computes {low} but the engine policy is {self.policy!r}")
            n = (self._fp8_weight if low == "fp8" else self._fp4_weight)(w_name, trans_b)[2]
            st, bmode = self._gemm_epi_state(node, bias_name, act, m, n, tuple(lead) + (n,))
            lower = self._gemm_fp8 if low == "fp8" else self._gemm_w4a16
            self.vals[st.final] = lower(node, a, w_name, trans_b, st, alpha, beta, bmode, tuple(lead) + (n,))
            return
        code = self.mm_code
        in_dtype = np.dtype(np.float32) if code == _lib.F32 else self.act_dtype
        w, n, kw = self._packed_weight_nk(w_name, trans_b, in_dtype)
        if kw != k or w.shape[1] != k:
            raise NotImplementedError(f"GEMM {node.id}: K={k} (weight K={kw}) needs padding for 16-bit MFMA")
        out_shape = tuple(lead) + (n,)
        st, bmode = self._gemm_epi_state(node, bias_name, act, m, n, out_shape)
        a2 = a if (a.dense and a.dtype == in_dtype) else self._dense(a, in_dtype)
        out = self._new(out_shape, self._out_dtype(st.final))
        self._finish_residual(st, out)
        mm = code
        if code == _lib.F32:
            splits = self._splitk(m, n, k)
        else:  # 16-bit: 128x128 tiles, K tiles of 64
            splits = self._splitk(m, n, k, vec=64, tile=128, min_k=64)
        if splits > 1:
            self._gemm_splitk(node, a2, w, out, st, m, n, k, splits, alpha, beta, bmode, in_code=code)
            return

        def build(r, a2=a2, w=w, out=out, st=st, m=m, n=n, k=k):
            g = _lib.GemmArgs()
            g.a, g.b, g.out = self._ptr(a2, r), self._ptr(w, r), self._ptr(out, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, k, k, k, n, 1
            g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, mm, dtype_code(out.dtype)
            self._fill_epi(g.epi, st, r, alpha, beta, bmode)
            return g
        self._emit(f"gemm:{node.op_type}", build, [a2, w] + self._epi_reads(st), [out], flops=2.0 * m * n * k,
                   info=f"M={m} N={n} K={k}")
        if mm != _lib.F32:
            self._note_row_max_site(st, out, m, n, alpha, beta, bmode)
        self.vals[st.final] = out

    def _splitk(self, m: int, n: int, k: int, vec: int = 4, tile: int = 64, min_k: int = 32) -> int:
        """K splits for a GEMM whose tile x tile output tiles cannot fill two
        blocks per CU (fp32: 64x64 tiles; 16-bit: 128x128): the largest split
        with K/split a multiple of `vec`, at least `min_k` deep, and at most
        two blocks per CU in total (1 = no split)."""
        tiles = -(-m // tile) * -(-n // tile)
        target = 2 * self._cus
        if 2 * tiles > target or k < 128:
            return 1
        best = 1
        for s in range(2, 65):
            if tiles * s > target:
                break
            if k % s == 0 and (k // s) % vec == 0 and k // s >= min_k:
                best = s
        return best

    def _gemm_splitk(self, node, a2: Val, w: Val, out: Val, st: "_Epi", m: int, n: int, k: int, splits: int,
                     alpha: float, beta: float, bmode, in_code: int = _lib.F32) -> None:
        """Split-K: `splits` batched partial GEMMs over K/splits each into an fp32
        workspace (fp32 accumulation for 16-bit operands too), then
        c3h_gemm_splitk_reduce (fixed summation order + epilogue)."""
        ks = k // splits
        part = self._new((splits, m, n), np.float32)

        def gbuild(r, a2=a2, w=w, part=part):
            g = _lib.GemmArgs()
            g.a, g.b, g.out = self._ptr(a2, r), self._ptr(w, r), self._ptr(part, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, ks, k, k, n, splits
            g.stride_a, g.stride_b, g.stride_out = ks, ks, m * n
            g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, in_code, _lib.F32
            g.epi.alpha, g.epi.beta = 1.0, 1.0
            return g
        self._emit(f"gemm:{node.op_type}", gbuild, [a2, w], [part], flops=2.0 * m * n * k,
                   info=f"M={m} N={n} K={k} in {splits} K splits")

        def rbuild(r, part=part, out=out, st=st):
            g = _lib.SplitKArgs()
            g.partial, g.out = self._ptr(part, r), self._ptr(out, r)
            g.m, g.n, g.ldo, g.splits, g.out_dtype = m, n, n, splits, dtype_code(out.dtype)
            self._fill_epi(g.epi, st, r, alpha, beta, bmode)
            return g
        self._emit("splitk_reduce", rbuild, [part] + self._epi_reads(st), [out])
        self.vals[st.final] = out

    def _op_FusedGemmEpilogue(self, node):
        a = self._get(node.inputs[0])
        fa = node.attributes.get("_flatten_axis")
        if fa is not None:
            ax = int(fa) + (len(a.shape) if int(fa) < 0 else 0)
            a = self._reshape_val(a, (math.prod(a.shape[:ax]), math.prod(a.shape[ax:])))
        if int(node.attributes.get("transA", 0)):
            a = self._dense(self._transpose_val(a, [1, 0]))
        act = 1 if node.attributes.get("_activation") == "Relu" else 0
        self._gemm_node(node, a, node.inputs[1], int(node.attributes.get("transB", 0)),
                        node.inputs[2] if len(node.inputs) > 2 else None, float(node.attributes.get("alpha", 1.0)),
                        float(node.attributes.get("beta", 1.0)), act, (a.shape[0],))

    def _op_FusedMatMulBias(self, node):
        a = self._get(node.inputs[0])
        self._gemm_node(node, a, node.inputs[1], 0, node.inputs[2], 1.0, 1.0, 0, a.shape[:-1])

    def _op_MatMul(self, node):
        pending = self.__dict__.get("_pending_attn", {})
        if node.inputs[0] in pending:
            scores, mask = pending.pop(node.inputs[0])
            self._flash(scores, node, mask)
            return
        a, b = self._get(node.inputs[0]), node.inputs[1]
        if b in self.weights_src and self._weight_host(b).ndim == 2:
            self._gemm_node(node, a, b, 0, None, 1.0, 1.0, 0, a.shape[:-1])
            return
        self._generic_matmul(node)

    def _generic_matmul(self, node):
        """Activation x activation MatMul through the fp32 batched GEMM."""
        a, b = self._dense(self._get(node.inputs[0]), np.float32), self._dense(self._get(node.inputs[1]), np.float32)
        m, k = a.shape[-2:]
        n = b.shape[-1]
        bs = E.broadcast_shape(a.shape[:-2], b.shape[:-2])
        if a.shape[:-2] != bs or b.shape[:-2] != bs:
            raise NotImplementedError("broadcast batched MatMul in the compiled engine")
        out = self._new(bs + (m, n), np.float32)
        nb = math.prod(bs)

        def build(r, a=a, b=b, out=out):
            g = _lib.GemmArgs()
            g.a, g.b, g.out = self._ptr(a, r), self._ptr(b, r), self._ptr(out, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, k, k, n, n, nb
            g.stride_a, g.stride_b, g.stride_out = m * k, k * n, m * n
            g.in_dtype, g.out_dtype = _lib.F32, _lib.F32
            g.epi.alpha, g.epi.beta = 1.0, 1.0
            return g
        self._emit("gemm:batched", build, [a, b], [out], flops=2.0 * nb * m * n * k)
        od = self._out_dtype(node.outputs[0])
        self.vals[node.outputs[0]] = out if od == np.float32 else self._dense(out, od)

    # -- convolution ----------------------------------------------------------------------------
    def _nhwc_input(self, x: Val, conv_dtype, c_pack: int) -> Val:
        """x as NHWC with channel stride c_pack in conv_dtype."""
        if x.layout == "nhwc" and x.c_stride == c_pack and x.dtype == conv_dtype:
            return x
        if x.layout == "nhwc":
            x = self._dense(x)
        src = x if x.dense else self._dense(x)
        n, c, h, w = src.shape
        out = self._new((n, c, h, w), conv_dtype, "nhwc", c_pack)

        def build(r, src=src, out=out):
            a = _lib.LayoutArgs()
            a.in_, a.out, a.n, a.c, a.h, a.w = self._ptr(src, r), self._ptr(out, r), n, c, h, w
            a.c_pad, a.direction, a.in_dtype, a.out_dtype = c_pack, 0, dtype_code(src.dtype), dtype_code(out.dtype)
            return a
        self._emit("layout", build, [src], [out])
        return out

    def _conv(self, node, x_name: str, w_name: str, bias_name: Optional[str], act: int,
              residual_name: Optional[str]) -> None:
        x = self._get(x_name)
        w_host = self._weight_host(w_name).astype(np.float32)
        o, cin, kh, kw = w_host.shape
        if int(node.attributes.get("group", 1)) != 1:
            raise NotImplementedError("grouped Conv in the compiled engine")
        n = x.shape[0]
        kh_, kw_, sh, sw, dh, dw, pads, ho, wo = E.conv_geometry(x.shape, w_host.shape, node.attributes)
        fp32 = self.mm_code == _lib.F32
        conv_dtype = np.dtype(np.float32) if fp32 else self.act_dtype
        narrow = (not fp32) and cin < 8
        if fp32:
            c_pack = (cin + 3) // 4 * 4
            kw_pack, k_stride = kw, kh * kw * c_pack
        elif narrow:
            c_pack, kw_pack = 4, (kw + 7) // 8 * 8
            k_stride = kh * kw_pack * 4
        else:
            c_pack = (cin + 7) // 8 * 8
            kw_pack = kw
            k_stride = (kh * kw * c_pack + 31) // 32 * 32
        wkey = (w_name, c_pack, kw_pack, k_stride, str(conv_dtype))
        wcache = self.__dict__.setdefault("_convw", {})
        if wkey not in wcache:
            src = self.weights_src[w_name]
            src_dev = src if isinstance(src, DeviceArray) else DeviceArray.from_host(w_host)
            packed = E.pack_conv_weight(src_dev, c_pack, kw_pack, k_stride, out_dtype=conv_dtype)
            wcache[wkey] = Val(packed.shape, packed.dtype, self._persist(packed))
            self._note_weight_store(w_name, conv_dtype)
        wv = wcache[wkey]
        if narrow and residual_name is None and self._stem_pool(node, x, wv, bias_name, act, cin, o, kh, kw, sh, sw,
                                                                  dh, dw, pads, ho, wo, k_stride):
            return
        xin = self._nhwc_input(x, conv_dtype, c_pack)
        out_shape = (n, o, ho, wo)
        st = _Epi(bias=self._bias_val(bias_name), act=act)
        if residual_name is not None:
            st.residual = self._get(residual_name)
        st = self._absorb_tail(node.outputs[0], out_shape, st)
        out = self._new(out_shape, self._out_dtype(st.final), "nhwc", o)
        self._finish_residual(st, out)
        code = dtype_code(conv_dtype)

        def build(r, xin=xin, wv=wv, out=out, st=st):
            a = _lib.ConvArgs()
            a.x, a.w, a.out = self._ptr(xin, r), self._ptr(wv, r), self._ptr(out, r)
            a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, cin, xin.shape[2], xin.shape[3], c_pack, c_pack, o
            a.kh, a.kw, a.sh, a.sw = kh, kw, sh, sw
            a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = pads[0], pads[1], dh, dw, ho, wo
            a.out_layout, a.in_dtype, a.out_dtype = 1, code, dtype_code(out.dtype)
            self._fill_epi(a.epi, st, r)
            return a
        self._emit("conv", build, [xin, wv] + self._epi_reads(st), [out],
                   flops=2.0 * n * ho * wo * o * cin * kh * kw,
                   info=f"{kh}x{kw}/{sh} {cin}->{o} {ho}x{wo}: M={n * ho * wo} N={o} K={cin * kh * kw}")
        self.vals[st.final] = out

    def _stem_pool(self, node, x: Val, wv: Val, bias_name, act, cin, o, kh, kw, sh, sw, dh, dw, pads, ho, wo,
                   k_stride) -> bool:
        """Conv 7x7/2 (c <= 3 -> 64) [+ ReLU] -> MaxPool 3x3/2 as one c3h_conv_stem_pool launch.

        Taken when the conv reads an NCHW tensor and its only consumer is the
        pool; the launch reads the NCHW input directly (no layout pass) and
        keeps the conv output in LDS.  Results equal the unfused chain."""
        if not self.fuse_stem or x.layout != "dense" or not x.dense or x.dtype not in (
                np.float32, np.float16) and x.dtype != self.act_dtype:
            return False
        if (cin > 3 or o != 64 or (kh, kw, sh, sw, dh, dw) != (7, 7, 2, 2, 1, 1) or tuple(pads[:2]) != (3, 3)
                or k_stride != 224 or act not in (0, 1)):
            return False
        pool, relu_node = self._single_consumer(node.outputs[0]), None
        if pool is not None and pool.op_type == "Relu" and act == 0:  # an unfused Relu between conv and pool
            relu_node, act = pool, 1
            pool = self._single_consumer(relu_node.outputs[0])
        if pool is None or pool.op_type != "MaxPool" or int(pool.attributes.get("ceil_mode", 0)):
            return False
        pk = list(pool.attributes.get("kernel_shape", []))
        pst = list(pool.attributes.get("strides", [1, 1]))
        pdl = list(pool.attributes.get("dilations", [1, 1]))
        ppads = list(pool.attributes.get("pads", [0, 0, 0, 0]))
        if pk != [3, 3] or pst != [2, 2] or pdl != [1, 1] or ppads[:2] != [1, 1] or pool.attributes.get("auto_pad",
                                                                                                        "NOTSET") != "NOTSET":
            return False
        n, _, h, w = x.shape
        _, _, _, _, _, _, _, po, qo = E.conv_geometry((n, o, ho, wo), (0, 0, 3, 3), pool.attributes)
        if not (2 * (po - 1) < ho and 2 * (qo - 1) < wo):
            return False
        out = self._new((n, o, po, qo), self.act_dtype, "nhwc", o)
        bias = self._bias_val(bias_name)

        def build(r, x=x, wv=wv, bias=bias, out=out):
            a = _lib.ConvPoolArgs()
            a.x, a.w, a.out = self._ptr(x, r), self._ptr(wv, r), self._ptr(out, r)
            a.bias = self._ptr(bias, r) if bias is not None else None
            a.n, a.c, a.h, a.w_, a.o, a.k_stride = n, cin, h, w, o, k_stride
            a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.ho, a.wo = kh, kw, sh, sw, 3, 3, ho, wo
            a.pkh, a.pkw, a.psh, a.psw, a.ppad_top, a.ppad_left, a.po, a.qo = 3, 3, 2, 2, 1, 1, po, qo
            a.relu, a.in_dtype, a.mm_dtype = int(act == 1), dtype_code(x.dtype), self.mm_code
            return a
        self._emit("conv:stem_pool", build, [x, wv] + ([bias] if bias is not None else []), [out],
                   flops=2.0 * n * ho * wo * o * cin * kh * kw,
                   info=f"{kh}x{kw}/{sh} {cin}->{o} {ho}x{wo} + pool -> {po}x{qo}: M={n * ho * wo} N={o} "
                        f"K={cin * kh * kw}")
        self.consumed.add(pool.id)
        if relu_node is not None:
            self.consumed.add(relu_node.id)
        self.vals[pool.outputs[0]] = out
        return True

    def _op_Conv(self, node):
        self._conv(node, node.inputs[0], node.inputs[1], node.inputs[2] if len(node.inputs) > 2 else None, 0, None)

    def _op_FusedConv2dBatchNorm(self, node):
        if not node.attributes.get("bn_folded"):
            raise NotImplementedError("compiled engine expects folded Conv+BN")
        self._conv(node, node.inputs[0], node.inputs[1], node.inputs[2] if len(node.inputs) > 2 else None, 0, None)

    def _op_FusedConvActivation(self, node):
        self._conv(node, node.inputs[0], node.inputs[1], node.inputs[2] if len(node.inputs) > 2 else None, 1, None)

    def _op_FusedConvResidualActivation(self, node):
        ri = int(node.attributes["_residual_input_index"])
        ins = node.inputs[:ri]
        self._conv(node, ins[0], ins[1], ins[2] if len(ins) > 2 else None, 1, node.inputs[ri])

    def _op_GlobalAveragePool(self, node):
        x = self._get(node.inputs[0])
        n, c = x.shape[:2]
        hw = math.prod(x.shape[2:])
        out = self._new((n, c) + (1,) * (len(x.shape) - 2), self._out_dtype(node.outputs[0]))
        if x.layout == "nhwc":
            src, outer, red, inner = x, n, hw, x.c_stride
            if x.c_stride != c:
                raise NotImplementedError("GAP over padded channels")
        else:
            src = x if x.dense else self._dense(x)
            outer, red, inner = n * c, hw, 1

        def build(r, src=src, out=out):
            a = _lib.ReduceArgs()
            a.in_, a.out, a.outer, a.reduce, a.inner = self._ptr(src, r), self._ptr(out, r), outer, red, inner
            a.kind, a.in_dtype, a.out_dtype = 2, dtype_code(src.dtype), dtype_code(out.dtype)
            return a
        self._emit("gap", build, [src], [out])
        self.vals[node.outputs[0]] = out

    def _op_MaxPool(self, node):
        x = self._get(node.inputs[0])
        if int(node.attributes.get("ceil_mode", 0)):
            raise NotImplementedError("MaxPool ceil_mode=1")
        kh, kw, sh, sw, dh, dw, pads, ho, wo = E.conv_geometry(x.shape, (0, 0) + tuple(node.attributes["kernel_shape"]),
                                                               node.attributes)
        n, c, h, w = x.shape
        if x.layout == "nhwc":
            out = self._new((n, c, ho, wo), x.dtype, "nhwc", x.c_stride)
            layout, cs = 1, x.c_stride
        else:
            x = x if x.dense else self._dense(x)
            out = self._new((n, c, ho, wo), x.dtype)
            layout, cs = 0, c

        def build(r, x=x, out=out):
            a = _lib.PoolArgs()
            a.x, a.out, a.n, a.c, a.h, a.w = self._ptr(x, r), self._ptr(out, r), n, c, h, w
            a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw = kh, kw, sh, sw, pads[0], pads[1], dh, dw
            a.ho, a.wo, a.layout, a.c_stride, a.dtype = ho, wo, layout, cs, dtype_code(x.dtype)
            return a
        self._emit("maxpool", build, [x], [out])
        self.vals[node.outputs[0]] = out

    # -- normalization / softmax / gather ----------------------------------------------------------
    def _layernorm(self, node, x: Val, residual: Optional[Val], scale_name: str, bias_name: Optional[str]) -> None:
        axis = int(node.attributes.get("axis", -1))
        axis = axis + len(x.shape) if axis < 0 else axis
        cols = math.prod(x.shape[axis:])
        rows = x.size // cols
        x = x if x.dense else self._dense(x)
        if residual is not None:
            residual = residual if (residual.dense and residual.dtype == x.dtype) else self._dense(residual, x.dtype)
        scale = self._weight_val(scale_name, np.float32)
        bias = self._weight_val(bias_name, np.float32) if bias_name else None
        eps = float(node.attributes.get("epsilon", 1e-5))
        # A QuantizeLinear that is the LayerNorm's only consumer runs in the same
        # launch (W8A8): int8 codes of the activation-type LayerNorm output.
        quant = self._fusable_quantize(node.outputs[0], cols, max_cols=LN_QUANT_MAX_COLS)
        ln_dtype = self._out_dtype(node.outputs[0])
        if quant is not None and ln_dtype != x.dtype:
            quant = None
        out = self._new(x.shape, np.int8 if quant is not None else ln_dtype)
        qscale, qzero = (quant[1], quant[2]) if quant is not None else (1.0, 0)

        def build(r, x=x, residual=residual, out=out, scale=scale, bias=bias):
            a = _lib.LayerNormArgs()
            a.x, a.residual = self._ptr(x, r), self._ptr(residual, r) if residual is not None else None
            a.scale, a.bias = self._ptr(scale, r), self._ptr(bias, r) if bias is not None else None
            a.out, a.mean_out, a.invstd_out = self._ptr(out, r), None, None
            a.rows, a.cols, a.epsilon, a.x_dtype, a.out_dtype = rows, cols, eps, dtype_code(x.dtype), dtype_code(out.dtype)
            a.out_scale, a.out_zero = qscale, qzero
            return a
        self._emit("layernorm_q" if quant is not None else "layernorm", build,
                   [x, scale] + ([bias] if bias else []) + ([residual] if residual else []), [out])
        if quant is not None:
            self.consumed.add(quant[0].id)
            self._rounded[node.outputs[0]] = _DTYPE_NAME[ln_dtype]
            self.vals[quant[0].outputs[0]] = out
        else:
            self.vals[node.outputs[0]] = out

    def _fusable_quantize(self, tensor: str, cols: int, max_cols: Optional[int] = None):
        """(QuantizeLinear node, scale, zero point) when `tensor`'s only consumer
        is a QuantizeLinear with a constant scalar scale and zero point that
        the producing launch can apply (not a graph output), else None.

        Mirrors the C entry points' preconditions, so a fused form that
        compiles also launches: cols % 8 == 0 (and cols <= max_cols for the
        LayerNorm form, c3h_layernorm's vector path), a positive normal fp32
        scale (quant_scale_ok: 2^-126 <= scale <= FLT_MAX) and an int8 zero
        point.  Anything else keeps the unfused pair."""
        q = self._single_consumer(tensor)
        if q is None or q.op_type != "QuantizeLinear" or q.id in self.consumed or self._is_output(tensor) or \
                cols % 8 or q.inputs[0] != tensor or (max_cols is not None and cols > max_cols):
            return None
        scale = self._scalar_const(q.inputs[1])
        zero = self._scalar_const(q.inputs[2]) if len(q.inputs) > 2 and q.inputs[2] else 0
        if scale is None or not quant_scale_ok(scale) or zero is None or zero != int(zero) or \
                not -128 <= int(zero) <= 127:
            return None
        return q, float(np.float32(scale)), int(zero)

    def _op_FusedLayerNormalization(self, node):
        self._layernorm(node, self._get(node.inputs[0]), None, node.inputs[1],
                        node.inputs[2] if len(node.inputs) > 2 else None)

    def _op_LayerNormalization(self, node):
        if len([o for o in node.outputs if o]) != 1:
            raise NotImplementedError("LayerNormalization with auxiliary outputs in the compiled engine")
        self._op_FusedLayerNormalization(node)

    def _op_FusedResidualNorm(self, node):
        self._layernorm(node, self._get(node.inputs[0]), self._get(node.inputs[1]), node.inputs[2],
                        node.inputs[3] if len(node.inputs) > 3 else None)

    def _softmax(self, node):
        x = self._get(node.inputs[0])
        x = x if x.dense else self._dense(x)
        axis = int(node.attributes.get("axis", -1))
        axis = axis + len(x.shape) if axis < 0 else axis
        out = self._new(x.shape, self._out_dtype(node.outputs[0]))

        def build(r, x=x, out=out):
            a = _lib.SoftmaxArgs()
            a.in_, a.out = self._ptr(x, r), self._ptr(out, r)
            a.outer, a.axis, a.inner = math.prod(x.shape[:axis]), x.shape[axis], math.prod(x.shape[axis + 1:])
            a.in_dtype, a.out_dtype = dtype_code(x.dtype), dtype_code(out.dtype)
            return a
        self._emit("softmax", build, [x], [out])
        self.vals[node.outputs[0]] = out

    _op_FusedSoftmaxDropout = _softmax
    _op_Softmax = _softmax

    def _op_Gather(self, node):
        data_name, idx = node.inputs[0], self._get(node.inputs[1])
        axis = int(node.attributes.get("axis", 0))
        if data_name in self.weights_src:
            data = self._weight_val(data_name, self.act_dtype if self._weight_host(data_name).dtype == np.float32
                                    else None)
        else:
            data = self._get(data_name)
            data = data if data.dense else self._dense(data)
        axis = axis + len(data.shape) if axis < 0 else axis
        shape = data.shape[:axis] + idx.shape + data.shape[axis + 1:]
        outer, adim, inner = math.prod(data.shape[:axis]), data.shape[axis], math.prod(data.shape[axis + 1:])
        add_node, addend = self._gather_addend(node, data, idx, axis, inner)
        final = add_node.outputs[0] if add_node is not None else node.outputs[0]
        od = self._out_dtype(final)
        out = self._new(shape, od if addend is not None else data.dtype)
        flag = self._error_flag()

        def build(r, data=data, idx=idx, out=out, addend=addend):
            a = _lib.GatherArgs()
            a.data, a.indices, a.out = self._ptr(data, r), self._ptr(idx, r), self._ptr(out, r)
            a.error_flag = flag.ptr
            a.outer, a.axis_dim, a.inner, a.n_indices, a.elem_bytes = outer, adim, inner, idx.size, data.dtype.itemsize
            if addend is not None:
                a.dtype, a.addend, a.addend_rows = dtype_code(out.dtype), self._ptr(addend, r), addend.size // inner
                a.addend_dtype = dtype_code(addend.dtype)
            return a
        self._emit("gather_add" if addend is not None else "gather", build,
                   [data, idx] + ([addend] if addend is not None else []), [out],
                   skip_bytes=[data], extra_bytes=outer * idx.size * inner * data.dtype.itemsize)
        if addend is not None:
            self.consumed.add(add_node.id)
        self.vals[final] = out if out.dtype == od else self._dense(out, od)

    def _gather_addend(self, node, data: Val, idx: Val, axis: int, inner: int):
        """(Add node, addend Val) when the gather's single consumer adds a
        constant table broadcast over the leading index dims -- the decoder's
        Gather(tok, ids) -> Add(., pos) -- so one launch does both; else (None, None).

        The table [rows, inner] must broadcast against [*idx.shape, inner] as
        trailing dims (rows = the product of idx's last dims), the gathered
        data must be 2-D (outer = 1).  The table is read in fp32, as the
        unfused Add reads it, and the gathered (stored-type) row plus the
        table is rounded once to the activation type: bit for bit the
        unfused Gather then Add."""
        add = self._single_consumer(node.outputs[0])
        if add is None or add.op_type != "Add" or add.id in self.consumed or axis != 0 or len(data.shape) != 2:
            return None, None
        others = [i for i in add.inputs if i != node.outputs[0]]
        if len(others) != 1 or others[0] not in self.weights_src or add.inputs.count(node.outputs[0]) != 1:
            return None, None
        w = self._weight_host(others[0])
        wshape = list(w.shape)
        while len(wshape) > 1 and wshape[0] == 1:
            wshape.pop(0)
        lead = wshape[:-1]
        if not wshape or wshape[-1] != inner or len(lead) > len(idx.shape) or \
                (lead and tuple(idx.shape[len(idx.shape) - len(lead):]) != tuple(lead)):
            return None, None
        od = self._out_dtype(add.outputs[0])
        if data.dtype != od or od not in (np.dtype(np.float32), BF16, np.dtype(np.float16)) or inner % 8 or \
                w.dtype != np.float32:
            return None, None
        return add, self._weight_val(others[0], np.float32)

    def _error_flag(self) -> DeviceArray:
        """A device int32 that kernels set to 1 on an invalid index (sticky until read)."""
        if getattr(self, "_errflag", None) is None:
            self._errflag = self._keep(DeviceArray.from_host(np.zeros(1, np.int32)))
        return self._errflag

    def read_value(self, name: str, rows: Optional[int] = None) -> np.ndarray:
        """Host copy of a value this program stores, in its logical (ONNX)
        shape and layout -- NHWC activations come back NCHW, strided views
        in their view order -- for the first `rows` entries of axis 0 (all if
        None).  16-bit floats are widened to float32; integers keep their type.
        Needs `keep_values=True` for anything but graph outputs and inputs
        (otherwise the memory may have been reused); synchronizes the device."""
        from ..device import bf16_to_f32

        v = self.vals[name]
        if v.buf is None:
            raise ValueError(f"value '{name}' is a host constant")
        if v.buf.kind == "slab" and not self.keep_values and name not in self.outputs:
            raise ValueError("read_value of an intermediate value needs keep_values=True")
        shape = list(v.shape)
        if rows is not None and shape:
            shape[0] = min(int(rows), shape[0])
        if math.prod(shape) == 0:
            return np.zeros(shape, np.float32)
        st = v.logical_strides()
        span = 1 + sum((d - 1) * s for d, s in zip(shape, st))
        base = self._resolve(v.buf) + v.offset * v.dtype.itemsize
        raw = DeviceArray(base, (span,), np.uint16 if v.dtype == BF16 else v.dtype, self.slab).get()
        item = raw.itemsize
        out = np.lib.stride_tricks.as_strided(raw, shape=shape, strides=[s * item for s in st]).copy()
        if v.dtype == BF16:
            return bf16_to_f32(out).reshape(shape)
        if v.dtype == np.float16:
            return out.astype(np.float32)
        return out

    def check_errors(self) -> None:
        """Raise IndexError if a kernel of this program saw an out-of-range
        index since the last check (the flag is cleared after reading).  A
        synchronous 4-byte read: call it after the program's stream has
        finished, outside any timed region."""
        flag = getattr(self, "_errflag", None)
        if flag is None:
            return
        if int(flag.get()[0]) != 0:
            flag.copy_from_host(np.zeros(1, np.int32))
            raise IndexError("Gather: an index is out of bounds for the gathered axis (ONNX Gather requires "
                             "-axis_dim <= index < axis_dim)")

    # -- attention ----------------------------------------------------------------------------------
    def _flash_mask(self, mask_name: str, s_q: int, s_k: int) -> Optional[Tuple[int, Optional[str]]]:
        """Classify a constant attention mask: (kind, name) with kind 0 none / 1 causal / 2 additive."""
        mask_host = self._host_value(mask_name)
        if mask_host is None:
            return None
        m2 = np.asarray(mask_host, np.float32)
        if m2.ndim < 2 or math.prod(m2.shape[:-2]) != 1 or m2.shape[-2:] != (s_q, s_k):
            return None
        m2 = m2.reshape(s_q, s_k)
        if not np.any(m2):
            return 0, None
        causal = np.triu(np.full((s_q, s_k), -np.inf, np.float32), 1)
        if np.array_equal(m2, causal):
            return 1, None
        return 2, mask_name

    def _op_FusedAttentionScores(self, node):
        """softmax(Q K^T / d + mask); with its P.V MatMul -> one flash-attention launch.

        The probabilities feed exactly one MatMul, so the scores node is held
        back until that MatMul is lowered (V's reshape/transpose views come
        in between) and both become one launch.
        """
        q, kt = self._get(node.inputs[0]), self._get(node.inputs[1])
        div = self._scalar_const(node.inputs[2])
        pv = self._single_consumer(node.outputs[0])
        ok = (pv is not None and pv.op_type == "MatMul" and pv.inputs[0] == node.outputs[0]
              and self.mm_code != _lib.F32 and q.shape[-1] == 64 and div is not None and div != 0.0
              and len(q.shape) == 4 and len(kt.shape) == 4 and q.shape[:2] == kt.shape[:2])
        mask = self._flash_mask(node.inputs[3], q.shape[2], kt.shape[3]) if ok else None
        if mask is None:
            self._attention_scores_materialized(node)
            return
        self.__dict__.setdefault("_pending_attn", {})[node.outputs[0]] = (node, mask)

    def _flash(self, node, pv, mask) -> None:
        q, kt, v = self._get(node.inputs[0]), self._get(node.inputs[1]), self._get(pv.inputs[1])
        div = self._scalar_const(node.inputs[2])
        mask_kind, mask_name = mask
        mask_val = self._weight_val(mask_name, np.float32) if mask_name else None
        b, h, s_q, d = q.shape
        s_k = kt.shape[3]
        if v.shape != (b, h, s_k, d):
            raise ValueError(f"attention: V shape {v.shape} does not match Q {q.shape} / K^T {kt.shape}")
        dt = self.act_dtype
        qv, kv, vv = (self._head_view(t, dt) for t in (q, self._transpose_val(kt, [0, 1, 3, 2]), v))
        # Stored in [B, S, H, D] order so the usual Transpose(0,2,1,3)+Reshape after it is a view.
        store = self._new((b, s_q, h, d), dt)
        ov = Val((b, h, s_q, d), dt, store.buf, 0, (s_q * h * d, d, h * d, 1))

        def build(r, qv=qv, kv=kv, vv=vv, store=store, mask_val=mask_val):
            a = _lib.FlashArgs()
            a.q, a.k, a.v = self._ptr(qv, r), self._ptr(kv, r), self._ptr(vv, r)
            a.mask = self._ptr(mask_val, r) if mask_val is not None else None
            a.out = self._ptr(store, r)
            a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim, a.dtype = b, h, s_q, s_k, d, dtype_code(dt)
            qs, ks, vs = qv.logical_strides(), kv.logical_strides(), vv.logical_strides()
            a.q_sb, a.q_sh, a.q_ss = qs[0], qs[1], qs[2]
            a.k_sb, a.k_sh, a.k_ss = ks[0], ks[1], ks[2]
            a.v_sb, a.v_sh, a.v_ss = vs[0], vs[1], vs[2]
            a.o_sb, a.o_sh, a.o_ss = s_q * h * d, d, h * d
            a.mask_ld, a.scale, a.mask_kind = s_k, 1.0 / div, mask_kind
            return a
        pairs = s_q * (s_q + 1) // 2 if (mask_kind == 1 and s_q == s_k) else s_q * s_k
        self._emit("flash", build, [qv, kv, vv] + ([mask_val] if mask_val else []), [store],
                   flops=4.0 * b * h * pairs * d)
        od = self._out_dtype(pv.outputs[0])
        self.vals[pv.outputs[0]] = ov if od == dt else self._dense(ov, od)

    def _head_view(self, t: Val, dt) -> Val:
        """A [B,H,S,D] view with unit D stride and 8-element aligned strides, in dtype dt."""
        st = t.logical_strides()
        if t.dtype == dt and st[3] == 1 and all(s % 8 == 0 for s in st[:3]) and t.offset % 8 == 0:
            return t
        return self._dense(t, dt)

    def _attention_scores_materialized(self, node):
        q, kt, div, mask = (self._dense(self._get(i), np.float32) for i in node.inputs[:4])
        q0, q1, rows, inner = q.shape
        k0, k1, _, cols = kt.shape
        mshape = [1] * (4 - len(mask.shape)) + list(mask.shape)
        out = self._new((max(q0, k0), max(q1, k1), rows, cols), np.float32)

        def build(r, q=q, kt=kt, div=div, mask=mask, out=out):
            a = _lib.AttnScoresArgs()
            a.q, a.kt, a.divisor, a.mask, a.out = (self._ptr(v, r) for v in (q, kt, div, mask, out))
            a.q0, a.q1, a.k0, a.k1, a.rows, a.cols, a.inner = q0, q1, k0, k1, rows, cols, inner
            a.m0, a.m1, a.m2, a.m3 = mshape
            a.in_dtype = _lib.F32
            return a
        self._emit("attn_scores", build, [q, kt, div, mask], [out],
                   flops=2.0 * max(q0, k0) * max(q1, k1) * rows * cols * inner)
        od = self._out_dtype(node.outputs[0])
        self.vals[node.outputs[0]] = out if od == np.float32 else self._dense(out, od)

    # -- ArgMax ------------------------------------------------------------------------------------------
    def _op_ArgMax(self, node):
        """First index of the maximum along the last axis (NumPy/ONNX tie rule), int64."""
        x = self._get(node.inputs[0])
        axis = int(node.attributes.get("axis", 0))
        axis = axis + len(x.shape) if axis < 0 else axis
        if axis != len(x.shape) - 1 or int(node.attributes.get("select_last_index", 0)):
            raise NotImplementedError("compiled ArgMax: last axis, first index only")
        x = x if x.dense else self._dense(x)
        cols = x.shape[-1]
        rows = x.size // cols
        keep = int(node.attributes.get("keepdims", 1))
        out = self._new(tuple(x.shape[:-1]) + ((1,) if keep else ()), np.int64)
        site = self.__dict__.get("_row_max_sites", {}).get(node.inputs[0])
        if site is not None and site[4] is x and site[2] == rows and site[3] == cols:
            # The producing GEMM also writes each row's 64-column block maxima
            # (its epilogue's row_max side output); the ArgMax finishes from
            # those and reads only the blocks that can hold the answer.
            gi, st = site[0], site[1]
            n_parts = -(-cols // 64)
            parts = self._new((rows, n_parts), np.int64)       # c3h_block_max entries (8 bytes)
            parts.buf.touch(gi)
            self.launch_rw[gi][1].append(parts.buf)
            self.launch_meta[gi]["bytes"] += parts.size * 8
            st.row_max = parts

            def fbuild(r, parts=parts, x=x, out=out):
                a = _lib.ArgmaxFinishArgs()
                a.parts, a.in_, a.out = self._ptr(parts, r), self._ptr(x, r), self._ptr(out, r)
                a.rows, a.cols, a.n_parts, a.ld, a.in_ld, a.in_dtype = rows, cols, n_parts, n_parts, cols, \
                    dtype_code(x.dtype)
                return a
            # algorithmic bytes: the block maxima, plus about one 64-column block of each row
            self._emit("argmax_finish", fbuild, [parts, x], [out], skip_bytes=[x],
                       extra_bytes=rows * 64 * x.dtype.itemsize)
            self.vals[node.outputs[0]] = out
            return

        def build(r, x=x, out=out):
            a = _lib.ArgmaxArgs()
            a.in_, a.out, a.rows, a.cols, a.in_dtype = self._ptr(x, r), self._ptr(out, r), rows, cols, \
                dtype_code(x.dtype)
            return a
        self._emit("argmax", build, [x], [out])
        self.vals[node.outputs[0]] = out

    # -- W8A8 -----------------------------------------------------------------------------------------
    def _op_QuantizeLinear(self, node):
        x = self._get(node.inputs[0])
        x = x if x.dense else self._dense(x)
        scale = self._scalar_const(node.inputs[1])
        zero = int(self._scalar_const(node.inputs[2])) if len(node.inputs) > 2 and node.inputs[2] else 0
        # c3h_quantize's precondition, checked here so the plan fails when it
        # is compiled rather than at its first launch
        if scale is None:
            raise NotImplementedError(f"QuantizeLinear '{node.id}': the compiled engine needs a constant scalar scale")
        if not quant_scale_ok(scale):
            raise ValueError(f"QuantizeLinear '{node.id}': scale {scale!r} is not a positive normal fp32 number")
        out = self._new(x.shape, np.int8)

        def build(r, x=x, out=out):
            a = _lib.QuantizeArgs()
            a.x, a.out, a.count, a.scale, a.zero_point, a.x_dtype = self._ptr(x, r), self._ptr(out, r), x.size, \
                scale, zero, dtype_code(x.dtype)
            return a
        self._emit("quantize", build, [x], [out])
        self.vals[node.outputs[0]] = out

    def _op_QLinearMatMul(self, node):
        """int8 GEMM; with its DequantizeLinear (+ bias/residual/GELU successors) as one launch.

        Fused form (qgemm mode 3): y = saturate(rne(acc * sa * sb[n] / sy)),
        then (y - 0) * sy and the epilogue -- the int8 value of the
        QLinearMatMul output is formed exactly as the unfused pair would.
        """
        a = self._get(node.inputs[0])
        a = a if a.dense else self._dense(a)
        sa, sy = self._scalar_const(node.inputs[1]), self._scalar_const(node.inputs[6])
        if sa is None or sy is None:
            raise NotImplementedError("QLinearMatMul with per-channel activation/output scales")
        for zi in (2, 5, 7):
            z = self._host_value(node.inputs[zi]) if len(node.inputs) > zi and node.inputs[zi] else None
            if z is not None and np.any(np.asarray(z) != 0):
                raise NotImplementedError("QLinearMatMul with nonzero zero points")
        wq = self._weight_host(node.inputs[3])
        if wq.ndim != 2 or wq.dtype != np.int8:
            raise NotImplementedError("QLinearMatMul needs a constant rank-2 int8 weight")
        k, n = wq.shape
        if a.shape[-1] != k:
            raise ValueError(f"QLinearMatMul {node.id}: inner dims {a.shape[-1]} vs {k}")
        cache = self.__dict__.setdefault("_qcache", {})
        if node.inputs[3] not in cache:
            bt = DeviceArray.from_host(np.ascontiguousarray(wq.T))
            sb = np.asarray(self._weight_host(node.inputs[4]), np.float32).reshape(-1)
            sbd = DeviceArray.from_host(np.full(n, sb[0], np.float32) if sb.size == 1 else sb)
            cache[node.inputs[3]] = (Val(bt.shape, bt.dtype, self._persist(bt)),
                                     Val(sbd.shape, sbd.dtype, self._persist(sbd)))
        bt, sbv = cache[node.inputs[3]]
        m = a.size // k
        shape = tuple(a.shape[:-1]) + (n,)
        deq = self._single_consumer(node.outputs[0])
        fuse = deq is not None and deq.op_type == "DequantizeLinear" and \
            self._scalar_const(deq.inputs[1]) == sy and \
            (len(deq.inputs) < 3 or not deq.inputs[2] or self._scalar_const(deq.inputs[2]) == 0)
        if not fuse:
            out = self._new(shape, np.int8)
            self._qgemm(a, bt, sbv, out, m, n, k, 1, sa, sy, _Epi())
            self.vals[node.outputs[0]] = out
            return
        self.consumed.add(deq.id)
        st = self._absorb_tail(deq.outputs[0], shape, _Epi())
        act_dtype = self._out_dtype(st.final)
        # A QuantizeLinear that is the epilogue output's only consumer (W8A8:
        # the GELU output ahead of FFN2) runs in the same launch: the value is
        # rounded to the activation type it would have been stored in, then
        # quantized -- the codes of the unfused pair.
        quant = self._fusable_quantize(st.final, n) if st.residual is None and not st.prog else None
        if quant is not None and act_dtype not in (np.float32, np.float16, BF16):
            quant = None
        out = self._new(shape, np.int8 if quant is not None else act_dtype)
        self._finish_residual(st, out)
        q = (dtype_code(act_dtype), quant[1], quant[2]) if quant is not None else None
        self._qgemm(a, bt, sbv, out, m, n, k, 3, sa, sy, st, q)
        if quant is None:
            self._note_row_max_site(st, out, m, n)
        if quant is not None:
            self.consumed.add(quant[0].id)
            self._rounded[st.final] = _DTYPE_NAME[act_dtype]
            self.vals[quant[0].outputs[0]] = out
        else:
            self.vals[st.final] = out

    def _qgemm(self, a, bt, sbv, out, m, n, k, mode, sa, sy, st: _Epi, quant=None):
        """quant: (act dtype code, scale, zero) of a QuantizeLinear applied to
        the epilogue's output (int8 `out`, modes 2 / 3)."""
        def build(r, a=a, bt=bt, sbv=sbv, out=out, st=st):
            g = _lib.QGemmArgs()
            g.a, g.b, g.out = self._ptr(a, r), self._ptr(bt, r), self._ptr(out, r)
            g.m, g.n, g.k, g.lda, g.ldb, g.ldo = m, n, k, k, k, n
            g.a_scale, g.y_scale, g.b_scale = sa, sy, self._ptr(sbv, r)
            g.y_zero, g.mode, g.out_dtype = 0, mode, dtype_code(out.dtype)
            if quant is not None:
                g.act_dtype, g.q_scale, g.q_zero = quant
            self._fill_epi(g.epi, st, r)
            return g
        self._emit("qgemm", build, [a, bt, sbv] + self._epi_reads(st), [out], flops=2.0 * m * n * k,
                   info=f"M={m} N={n} K={k}")

    def _op_DequantizeLinear(self, node):
        q = self._get(node.inputs[0])
        scale = self._scalar_const(node.inputs[1])
        zero = int(self._scalar_const(node.inputs[2])) if len(node.inputs) > 2 and node.inputs[2] else 0
        out = self._new(q.shape, self._out_dtype(node.outputs[0]))

        def build(r, q=q, out=out):
            a = _lib.DequantizeArgs()
            a.q, a.out, a.count, a.scale, a.zero_point, a.out_dtype = self._ptr(q, r), self._ptr(out, r), q.size, \
                scale, zero, dtype_code(out.dtype)
            return a
        self._emit("dequantize", build, [q], [out])
        self.vals[node.outputs[0]] = out


def _gelu_program_to_act(st: "_Epi") -> None:
    """Replace the decomposed-GELU program by the kernels' compiled GELU (act 2).

    The program Div(x, c0) -> Erf -> Add(., c1) -> Mul(x, .) -> Mul(., c2) is
    what the Div/Erf/Add/Mul/Mul chain of a GELU lowers to; act 2 evaluates
    the same five operations in the same order (Add and Mul operands may come
    in either order: they commute exactly), with the division and the erf
    each within an fp32 ulp or two of the correctly rounded ones.
    """
    if st.act or len(st.prog) != 5:
        return
    (o0, a0, b0, _), (o1, a1, _, _), (o2, a2, b2, _), (o3, a3, b3, _), (o4, a4, b4, _) = st.prog
    if [o0, o1, o2, o3, o4] != [_lib.EW_DIV, _lib.EW_ERF, _lib.EW_ADD, _lib.EW_MUL, _lib.EW_MUL]:
        return
    if a0 not in (0, 1) or b0 < 2 or a1 != 1:
        return
    if sorted((a2, b2))[0] != 1 or max(a2, b2) < 2:
        return
    if sorted((a3, b3)) != [0, 1]:
        return
    if sorted((a4, b4))[0] != 1 or max(a4, b4) < 2:
        return
    c = [st.imm[b0 - 2], st.imm[max(a2, b2) - 2], st.imm[max(a4, b4) - 2]]
    st.prog, st.imm, st.act = [], c, 2


def _reshape_strides(shape, strides, new_shape) -> Optional[Tuple[int, ...]]:
    """Strides of a no-copy reshape of a strided view, or None when a copy is needed.

    Size-1 dims are ignored; the remaining old and new dims are matched in
    groups of equal product, and each old group must be contiguous.
    """
    new_shape = tuple(int(d) for d in new_shape)
    if math.prod(shape) != math.prod(new_shape):
        raise ValueError(f"reshape {tuple(shape)} -> {new_shape}: element counts differ")
    if math.prod(new_shape) == 0:
        return tuple(E.dense_strides(new_shape))
    old = [(d, s) for d, s in zip(shape, strides) if d != 1]
    nz = [i for i, d in enumerate(new_shape) if d != 1]
    out = [0] * len(new_shape)
    oi = k = 0
    while k < len(nz):
        og, ng = oi, k
        op, npd = old[oi][0], new_shape[nz[k]]
        while op != npd:
            if op < npd:
                oi += 1
                op *= old[oi][0]
            else:
                k += 1
                npd *= new_shape[nz[k]]
        for j in range(og, oi):
            if old[j][1] != old[j + 1][1] * old[j + 1][0]:
                return None
        st = old[oi][1]
        for j in range(k, ng - 1, -1):
            out[nz[j]] = st
            st *= new_shape[nz[j]]
        oi += 1
        k += 1
    inner = 1
    for i in range(len(new_shape) - 1, -1, -1):  # size-1 dims: the dense-consistent stride
        if new_shape[i] == 1:
            out[i] = inner
        else:
            inner = out[i] * new_shape[i]
    return tuple(out)
