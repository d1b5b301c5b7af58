"""Operator library on DeviceArrays (counterpart of c35/engine.py).

Every ONNX op and C3.3 fused op the reference engine implements
(c35/engine.py:229-716 and 722-1445) is here as a launch of a libc3hip.so
kernel family on the current stream; there is no host-side numerical path.
Output placement follows the reference's `_planned_output` contract
(E:34-69) with one change: `attrs["_planned_output"]` may be any device
array of sufficient capacity (the executor passes the flat arena view) and
the result is written there directly - no temporary plus copy.
"""

from __future__ import annotations

import ctypes as C
import math
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import _lib
from ..device import BF16, DeviceArray, current_stream, dtype_code

F32 = np.dtype(np.float32)


# ---------------------------------------------------------------- helpers
def _planned(attrs: Dict[str, Any], shape: Sequence[int], dtype=np.float32) -> DeviceArray:
    """The output array: a view into attrs['_planned_output'] or a new allocation."""
    shape = tuple(int(d) for d in shape)
    out = attrs.get("_planned_output")
    if out is None:
        return DeviceArray.empty(shape, dtype)
    if not isinstance(out, DeviceArray):
        raise TypeError("_planned_output must be a DeviceArray")
    need = math.prod(shape) * np.dtype(dtype).itemsize
    if out.nbytes < need:
        raise ValueError(f"Output arena too small: need {need} bytes, have {out.nbytes}")
    return DeviceArray(out.ptr, shape, dtype, out.owner)


def broadcast_shape(*shapes: Sequence[int]) -> Tuple[int, ...]:
    rank = max((len(s) for s in shapes), default=0)
    out = [1] * rank
    for s in shapes:
        padded = (1,) * (rank - len(s)) + tuple(int(d) for d in s)
        for i, d in enumerate(padded):
            if out[i] == 1:
                out[i] = d
            elif d not in (1, out[i]):
                raise ValueError(f"Shapes {shapes} are not broadcastable")
    return tuple(out)


def broadcast_strides(shape: Sequence[int], out_shape: Sequence[int]) -> List[int]:
    """Element strides of a dense `shape` read under broadcasting to `out_shape`."""
    rank = len(out_shape)
    padded = (1,) * (rank - len(shape)) + tuple(int(d) for d in shape)
    strides = [0] * rank
    acc = 1
    for i in range(rank - 1, -1, -1):
        strides[i] = 0 if (padded[i] == 1 and out_shape[i] != 1) else acc
        acc *= padded[i]
    return strides


def _as_float(x: DeviceArray) -> DeviceArray:
    return x


_EW_BINARY = {"Add": _lib.EW_ADD, "Sub": _lib.EW_SUB, "Mul": _lib.EW_MUL, "Div": _lib.EW_DIV}
_EW_UNARY_CHAIN = {"Relu": _lib.EW_RELU, "Erf": _lib.EW_ERF, "Sqrt": _lib.EW_SQRT, "Exp": _lib.EW_EXP}


def ew_args(inputs: Sequence[DeviceArray], program: Sequence[Tuple[int, int, int, float]],
            out: DeviceArray, out_shape: Sequence[int]) -> _lib.EwArgs:
    """Build c3h_ew_args for `program` = [(opcode, reg_a, reg_b, imm), ...]."""
    if len(inputs) > _lib.EW_MAX_IN or len(program) > _lib.EW_MAX_INST or len(out_shape) > _lib.MAX_RANK:
        raise ValueError("elementwise program exceeds the kernel's limits")
    a = _lib.EwArgs()
    for j, x in enumerate(inputs):
        a.in_[j] = x.ptr
        a.in_dtype[j] = x.code
        for d, s in enumerate(broadcast_strides(x.shape, out_shape)):
            a.stride[j][d] = s
    a.out = out.ptr
    a.out_dtype = out.code
    a.rank = len(out_shape)
    for d, s in enumerate(out_shape):
        a.shape[d] = int(s)
    a.n_in = len(inputs)
    a.n_inst = len(program)
    for i, (op, ra, rb, imm) in enumerate(program):
        a.inst[i].op, a.inst[i].a, a.inst[i].b, a.inst[i].imm = op, ra, rb, float(imm)
    return a


def run_ew(inputs: Sequence[DeviceArray], program, attrs: Dict[str, Any], out_dtype=np.float32) -> DeviceArray:
    shape = broadcast_shape(*(x.shape for x in inputs))
    out = _planned(attrs, shape, out_dtype)
    if out.size:
        _lib.launch(ew_args(inputs, program, out, shape), current_stream())
    return out


def strided_copy(x: DeviceArray, out: DeviceArray, shape: Sequence[int], strides: Sequence[int],
                 offset: int = 0) -> None:
    a = _lib.CopyArgs()
    a.in_, a.out, a.elem_bytes, a.rank = x.ptr, out.ptr, x.itemsize, len(shape)
    for d, (n, s) in enumerate(zip(shape, strides)):
        a.shape[d], a.in_stride[d] = int(n), int(s)
    a.in_offset = int(offset)
    if math.prod(shape):
        _lib.launch(a, current_stream())


def dense_strides(shape: Sequence[int]) -> List[int]:
    out, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        out[i] = acc
        acc *= int(shape[i])
    return out


def copy_into(x: DeviceArray, out: DeviceArray) -> DeviceArray:
    if x.nbytes != out.nbytes:
        raise ValueError("copy size mismatch")
    if x.ptr != out.ptr and x.nbytes:
        _lib.check(_lib.lib().c3h_memcpy_d2d_async(out.ptr, x.ptr, x.nbytes, current_stream()), "d2d")
    return out


def cast_into(x: DeviceArray, out: DeviceArray) -> DeviceArray:
    if x.dtype == out.dtype:
        return copy_into(x, out)
    a = _lib.CastArgs()
    a.in_, a.out, a.count, a.in_dtype, a.out_dtype = x.ptr, out.ptr, x.size, x.code, out.code
    if x.size:
        _lib.launch(a, current_stream())
    return out


def to_host_ints(x: DeviceArray) -> List[int]:
    """Control metadata (shape tensors) read back to the host, as the reference does (E:76)."""
    return [int(v) for v in x.get().reshape(-1).tolist()]


def epilogue(bias: Optional[DeviceArray] = None, bias_mode: int = 0, alpha: float = 1.0, beta: float = 1.0,
             act: int = 0, residual: Optional[DeviceArray] = None,
             program: Sequence[Tuple[int, int, int, float]] = (), imm: Sequence[float] = ()) -> _lib.Epilogue:
    e = _lib.Epilogue()
    e.bias = bias.ptr if bias is not None else None
    e.residual = residual.ptr if residual is not None else None
    e.alpha, e.beta, e.bias_mode, e.act = float(alpha), float(beta), int(bias_mode), int(act)
    e.n_imm = len(imm)
    for i, v in enumerate(imm):
        e.imm[i] = float(v)
    e.n_inst = len(program)
    for i, (op, ra, rb, iv) in enumerate(program):
        e.inst[i].op, e.inst[i].a, e.inst[i].b, e.inst[i].imm = op, ra, rb, float(iv)
    return e


def gemm(a: DeviceArray, b: DeviceArray, out: DeviceArray, m: int, n: int, k: int, lda: int, ldb: int, ldo: int,
         trans_a: int = 0, trans_b: int = 0, epi: Optional[_lib.Epilogue] = None, batch: int = 1,
         stride_a: int = 0, stride_b: int = 0, stride_out: int = 0, stride_bias: int = 0,
         stride_res: int = 0, in_dtype: Optional[int] = None) -> None:
    g = _lib.GemmArgs()
    g.a, g.b, g.out = a.ptr, b.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo = m, n, k, lda, ldb, ldo
    g.batch, g.stride_a, g.stride_b, g.stride_out = batch, stride_a, stride_b, stride_out
    g.stride_bias, g.stride_res = stride_bias, stride_res
    g.trans_a, g.trans_b = trans_a, trans_b
    g.in_dtype = a.code if in_dtype is None else in_dtype
    g.out_dtype = out.code
    g.epi = epi if epi is not None else epilogue()
    _lib.launch(g, current_stream())


def gemm_splitk(g: _lib.GemmArgs, splits: int, workspace: DeviceArray) -> None:
    """c3h_gemm_splitk: the GEMM `g` cut along K into `splits` partial GEMMs
    in `workspace` (fp32 [splits, m, n]), then the ordered reduce + epilogue."""
    _lib.check(_lib.lib().c3h_gemm_splitk(C.byref(g), int(splits), workspace.ptr, workspace.nbytes,
                                          current_stream()), "c3h_gemm_splitk")


def _bias_mode(bias: Optional[DeviceArray], m: int, n: int) -> Tuple[int, int, int]:
    """(mode, rows, cols) of a Gemm C operand broadcast to [m, n] (E:771-793)."""
    if bias is None:
        return 0, 1, 1
    shape = list(bias.shape)
    while len(shape) > 2 and shape[0] == 1:
        shape.pop(0)
    if len(shape) == 0:
        rows, cols = 1, 1
    elif len(shape) == 1:
        rows, cols = 1, shape[0]
    elif len(shape) == 2:
        rows, cols = shape
    else:
        raise ValueError("Fused GEMM bias rank is not broadcastable")
    if rows not in (1, m) or cols not in (1, n):
        raise ValueError(f"Fused GEMM bias shape {bias.shape} cannot broadcast to {(m, n)}")
    mode = {(1, 1): 1, (1, n): 2, (m, 1): 3, (m, n): 4}.get((rows, cols))
    if rows == 1 and cols == 1:
        mode = 1
    elif rows == 1:
        mode = 2
    elif cols == 1:
        mode = 3
    else:
        mode = 4
    return mode, rows, cols


# ---------------------------------------------------------------- ONNX ops (E:229-716)
def op_flatten(inputs, attrs):
    x = inputs[0]
    axis = int(attrs.get("axis", 1))
    axis = axis + x.ndim if axis < 0 else axis
    if not 0 <= axis <= x.ndim:
        raise ValueError(f"Flatten axis {axis} is invalid for rank {x.ndim}")
    shape = (math.prod(x.shape[:axis]), math.prod(x.shape[axis:]))
    if attrs.get("_planned_output") is None:
        return x.reshape(shape)
    return copy_into(x.reshape(shape), _planned(attrs, shape, x.dtype))


def _execute_gemm_epilogue(inputs, attrs, matmul_semantics: bool):
    if len(inputs) < 2:
        raise ValueError("Fused GEMM requires A and B inputs")
    a, b = inputs[0], inputs[1]
    if b.ndim != 2:
        raise ValueError("Fused GEMM requires a rank-2 B input")
    fa = attrs.get("_flatten_axis")
    if fa is not None:
        ax = int(fa) + (a.ndim if int(fa) < 0 else 0)
        if not 0 <= ax <= a.ndim:
            raise ValueError("Fused GEMM Flatten axis is out of range")
        a = a.reshape(math.prod(a.shape[:ax]), math.prod(a.shape[ax:]))
    if matmul_semantics:
        if a.ndim < 2:
            raise ValueError("Fused MatMul+bias requires rank >= 2")
        lead = a.shape[:-1]
        a = a.reshape(-1, a.shape[-1])
        ta = tb = 0
    else:
        if a.ndim != 2:
            raise ValueError("Fused Gemm requires rank-2 A after Flatten")
        lead = ()
        ta, tb = int(attrs.get("transA", 0)), int(attrs.get("transB", 0))
        if ta not in (0, 1) or tb not in (0, 1):
            raise ValueError("Gemm transA and transB must be 0 or 1")
    m = a.shape[1] if ta else a.shape[0]
    k = a.shape[0] if ta else a.shape[1]
    bk = b.shape[1] if tb else b.shape[0]
    n = b.shape[0] if tb else b.shape[1]
    if k != bk:
        raise ValueError(f"Fused GEMM inner dimensions differ: {k} and {bk}")
    bias = inputs[2] if len(inputs) >= 3 else None
    mode, rows, cols = _bias_mode(bias, m, n)
    out = _planned(attrs, lead + (n,) if matmul_semantics else (m, n))
    act = 1 if attrs.get("_activation") == "Relu" else 0
    epi = epilogue(bias=bias, bias_mode=mode, alpha=float(attrs.get("alpha", 1.0)),
                   beta=float(attrs.get("beta", 1.0)), act=act)
    if mode == 4 and rows == m and cols == n:
        pass
    gemm(a, b, out, m, n, k, lda=a.shape[1], ldb=b.shape[1], ldo=n, trans_a=ta, trans_b=tb, epi=epi)
    return out


def op_gemm(inputs, attrs):
    a, b = inputs[0], inputs[1]
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("Gemm inputs A and B must both have rank 2")
    c = inputs[2] if len(inputs) >= 3 else None
    return _execute_gemm_epilogue([a, b] + ([c] if c is not None else []), attrs, matmul_semantics=False)


def op_relu(inputs, attrs):
    return run_ew([inputs[0]], [(_lib.EW_RELU, 0, 0, 0.0)], attrs)


def _binary(op: int):
    def fn(inputs, attrs):
        return run_ew([inputs[0], inputs[1]], [(op, 0, 1, 0.0)], attrs)
    return fn


op_add = _binary(_lib.EW_ADD)
op_sub = _binary(_lib.EW_SUB)
op_mul = _binary(_lib.EW_MUL)
op_div = _binary(_lib.EW_DIV)


def op_erf(inputs, attrs):
    """Unfused Erf uses the A&S 7.1.26 formula like the reference (E:653-659)."""
    return run_ew([inputs[0]], [(_lib.EW_ERF_AS, 0, 0, 0.0)], attrs)


def op_exp(inputs, attrs):
    return run_ew([inputs[0]], [(_lib.EW_EXP, 0, 0, 0.0)], attrs)


def op_sqrt(inputs, attrs):
    return run_ew([inputs[0]], [(_lib.EW_SQRT, 0, 0, 0.0)], attrs)


def op_reciprocal(inputs, attrs):
    return run_ew([inputs[0]], [(_lib.EW_RECIP, 0, 0, 0.0)], attrs)


def _contiguous_axes(axes: Sequence[int], ndim: int) -> bool:
    s = sorted(axes)
    return s == list(range(s[0], s[-1] + 1)) if s else True


def reduce(x: DeviceArray, axes: Sequence[int], keepdims: bool, kind: int, attrs) -> DeviceArray:
    """max (0) / sum (1) / mean (2) over a contiguous block of axes."""
    axes = sorted({a % x.ndim for a in axes}) if x.ndim else []
    if not _contiguous_axes(axes, x.ndim):
        raise NotImplementedError(f"reduction over non-adjacent axes {axes} is not supported")
    if axes:
        outer = math.prod(x.shape[:axes[0]])
        red = math.prod(x.shape[axes[0]:axes[-1] + 1])
        inner = math.prod(x.shape[axes[-1] + 1:])
    else:
        outer, red, inner = x.size, 1, 1
    shape = tuple(1 if i in axes else d for i, d in enumerate(x.shape)) if keepdims else \
        tuple(d for i, d in enumerate(x.shape) if i not in axes)
    out = _planned(attrs, shape)
    a = _lib.ReduceArgs()
    a.in_, a.out, a.outer, a.reduce, a.inner = x.ptr, out.ptr, outer, red, inner
    a.kind, a.in_dtype, a.out_dtype = kind, x.code, out.code
    if outer * inner:
        _lib.launch(a, current_stream())
    return out


def op_global_average_pool(inputs, attrs):
    x = inputs[0]
    return reduce(x, list(range(2, x.ndim)), True, 2, attrs)


_GATHER_FLAG: Optional[DeviceArray] = None


def gather_error_flag() -> DeviceArray:
    """The device int32 every engine gather sets to 1 on an out-of-range index."""
    global _GATHER_FLAG
    if _GATHER_FLAG is None:
        _GATHER_FLAG = DeviceArray.from_host(np.zeros(1, np.int32))
    return _GATHER_FLAG


def check_gather_errors() -> None:
    """Raise IndexError (as np.take does) if a gather since the last check saw
    an index outside [-axis_dim, axis_dim); clears the flag.  Synchronous."""
    if _GATHER_FLAG is not None and int(_GATHER_FLAG.get()[0]) != 0:
        _GATHER_FLAG.copy_from_host(np.zeros(1, np.int32))
        raise IndexError("Gather: an index is out of bounds for the gathered axis (ONNX Gather requires "
                         "-axis_dim <= index < axis_dim)")


def gather(x: DeviceArray, idx: DeviceArray, axis: int, attrs, out_dtype=None) -> DeviceArray:
    axis = axis + x.ndim if axis < 0 else axis
    if not 0 <= axis < x.ndim:
        raise ValueError(f"Gather axis {axis} is invalid for rank {x.ndim}")
    if idx.dtype != np.int64:
        raise TypeError("gather indices must be int64")
    shape = x.shape[:axis] + idx.shape + x.shape[axis + 1:]
    out_dtype = x.dtype if out_dtype is None else np.dtype(out_dtype)
    direct = out_dtype == x.dtype
    out = _planned(attrs, shape, out_dtype) if direct else DeviceArray.empty(shape, x.dtype)
    a = _lib.GatherArgs()
    a.data, a.indices, a.out, a.error_flag = x.ptr, idx.ptr, out.ptr, gather_error_flag().ptr
    a.outer, a.axis_dim, a.inner = math.prod(x.shape[:axis]), x.shape[axis], math.prod(x.shape[axis + 1:])
    a.n_indices, a.elem_bytes = idx.size, x.itemsize
    if out.size:
        _lib.launch(a, current_stream())
    if direct:
        return out
    return cast_into(out, _planned(attrs, shape, out_dtype))


def op_gather(inputs, attrs):
    return gather(inputs[0], inputs[1], int(attrs.get("axis", 0)), attrs)


def layer_norm(x: DeviceArray, scale: DeviceArray, bias: Optional[DeviceArray], axis: int, eps: float, attrs,
               residual: Optional[DeviceArray] = None, n_outputs: int = 1, out_dtype=None):
    axis = axis + x.ndim if axis < 0 else axis
    if not 0 <= axis < x.ndim:
        raise ValueError(f"LayerNormalization axis {axis} is invalid for rank {x.ndim}")
    cols = math.prod(x.shape[axis:])
    rows = x.size // cols if cols else 0
    if scale.size != cols:
        raise ValueError("LayerNormalization scale size does not match normalized shape")
    if bias is not None and bias.size != cols:
        raise ValueError("LayerNormalization bias size does not match normalized shape")
    out = _planned(attrs, x.shape, x.dtype if out_dtype is None else out_dtype)
    stat_shape = x.shape[:axis] + (1,) * (x.ndim - axis)
    mean = invstd = None
    if n_outputs >= 2:
        mean = _planned({"_planned_output": attrs.get("_planned_output_1")}, stat_shape) \
            if attrs.get("_planned_output_1") is not None else DeviceArray.empty(stat_shape, np.float32)
    if n_outputs >= 3:
        invstd = _planned({"_planned_output": attrs.get("_planned_output_2")}, stat_shape) \
            if attrs.get("_planned_output_2") is not None else DeviceArray.empty(stat_shape, np.float32)
    a = _lib.LayerNormArgs()
    a.x, a.residual, a.scale = x.ptr, residual.ptr if residual is not None else None, scale.ptr
    a.bias, a.out = bias.ptr if bias is not None else None, out.ptr
    a.mean_out, a.invstd_out = (mean.ptr if mean is not None else None), (invstd.ptr if invstd is not None else None)
    a.rows, a.cols, a.epsilon, a.x_dtype, a.out_dtype = rows, cols, float(eps), x.code, out.code
    if rows:
        _lib.launch(a, current_stream())
    if n_outputs == 1:
        return out
    return [out, mean] + ([invstd] if n_outputs == 3 else [])


def op_layer_normalization(inputs, attrs):
    n_out = int(attrs.get("_num_outputs", 1))
    if not 1 <= n_out <= 3:
        raise ValueError("LayerNormalization supports one to three outputs")
    return layer_norm(inputs[0], inputs[1], inputs[2] if len(inputs) > 2 else None, int(attrs.get("axis", -1)),
                      float(attrs.get("epsilon", 1e-5)), attrs, n_outputs=n_out)


def op_matmul(inputs, attrs):
    """ONNX MatMul with NumPy batch broadcasting (E:535-543)."""
    a, b = inputs[0], inputs[1]
    a2 = a.reshape(1, a.shape[0]) if a.ndim == 1 else a
    b2 = b.reshape(b.shape[0], 1) if b.ndim == 1 else b
    m, k = a2.shape[-2:]
    kb, n = b2.shape[-2:]
    if k != kb:
        raise ValueError(f"MatMul inner dimensions differ: {k} and {kb}")
    batch_shape = broadcast_shape(a2.shape[:-2], b2.shape[:-2])
    out_shape = batch_shape + (m, n)
    final_shape = list(out_shape)
    if a.ndim == 1:
        final_shape.pop(-2)
    if b.ndim == 1:
        final_shape.pop(-1)
    out = _planned(attrs, out_shape)
    alpha = float(attrs.get("alpha", 1.0))
    epi = epilogue(alpha=alpha)
    nb = math.prod(batch_shape)
    sa = broadcast_strides(a2.shape[:-2], batch_shape)
    sb = broadcast_strides(b2.shape[:-2], batch_shape)
    # Collapse to one batched launch when each operand's batch walk is a single stride.
    def single_stride(strides, shape, elems):
        eff = [(s, d) for s, d in zip(strides, shape) if d != 1]
        if not eff:
            return 0
        if all(s == 0 for s, _ in eff):
            return 0
        if all(s != 0 for s, _ in eff):
            return elems
        return None
    stride_a = single_stride(sa, batch_shape, m * k)
    stride_b = single_stride(sb, batch_shape, k * n)
    if nb <= 65535 and stride_a is not None and stride_b is not None:
        gemm(a2, b2, out, m, n, k, lda=k, ldb=n, ldo=n, epi=epi, batch=nb, stride_a=stride_a, stride_b=stride_b,
             stride_out=m * n)
    else:
        for idx in np.ndindex(*batch_shape):
            oa = sum(i * s for i, s in zip(idx, sa)) * m * k
            ob = sum(i * s for i, s in zip(idx, sb)) * k * n
            oo = int(np.ravel_multi_index(idx, batch_shape)) * m * n if batch_shape else 0
            gemm(a2.ravel().flat(oa, oa + m * k), b2.ravel().flat(ob, ob + k * n),
                 out.ravel().flat(oo, oo + m * n), m, n, k, lda=k, ldb=n, ldo=n, epi=epi)
    return out.reshape(final_shape)


def op_constant(inputs, attrs):
    raise RuntimeError("Constant nodes must be pre-loaded as weights")


def op_split(inputs, attrs):
    x = inputs[0]
    axis = int(attrs.get("axis", 0))
    axis = axis + x.ndim if axis < 0 else axis
    if not 0 <= axis < x.ndim:
        raise ValueError(f"Split axis {axis} is invalid for rank {x.ndim}")
    sizes_in = inputs[1] if len(inputs) > 1 else None
    if sizes_in is not None and sizes_in.size > 0:
        sizes = to_host_ints(sizes_in)
    elif attrs.get("split"):
        sizes = [int(s) for s in attrs["split"]]
    else:
        n_out = int(attrs.get("_num_outputs", 2))
        if n_out <= 0 or x.shape[axis] % n_out:
            raise ValueError("Equal Split requires a positive divisor of the axis size")
        sizes = [x.shape[axis] // n_out] * n_out
    n_out = int(attrs.get("_num_outputs", len(sizes)))
    if len(sizes) != n_out:
        raise ValueError("Split size count must equal the number of outputs")
    if any(s < 0 for s in sizes) or sum(sizes) != x.shape[axis]:
        raise ValueError("Split sizes must be non-negative and sum to the axis size")
    strides = dense_strides(x.shape)
    outs, start = [], 0
    planned = attrs.get("_planned_outputs") or [None] * n_out
    for i, size in enumerate(sizes):
        shape = x.shape[:axis] + (size,) + x.shape[axis + 1:]
        out = _planned({"_planned_output": planned[i]}, shape, x.dtype)
        strided_copy(x, out, shape, strides, offset=start * strides[axis])
        outs.append(out)
        start += size
    return outs


def resolve_reshape_shape(in_shape: Sequence[int], target_raw: Sequence[int], allowzero: int) -> Tuple[int, ...]:
    """ONNX Reshape target resolution (E:72-107)."""
    if allowzero not in (0, 1):
        raise ValueError("Reshape allowzero must be 0 or 1")
    if allowzero and 0 in target_raw and -1 in target_raw:
        raise ValueError("Reshape cannot combine a literal zero and -1 when allowzero=1")
    target, infer, known = [], None, 1
    for i, d in enumerate(int(v) for v in target_raw):
        if d == 0 and not allowzero:
            if i >= len(in_shape):
                raise ValueError("Reshape zero index exceeds input rank")
            d = int(in_shape[i])
        if d == -1:
            if infer is not None:
                raise ValueError("Reshape permits at most one inferred dimension")
            infer = i
            target.append(-1)
        else:
            if d < 0:
                raise ValueError("Reshape dimensions must be non-negative or -1")
            target.append(d)
            known *= d
    total = math.prod(int(d) for d in in_shape)
    if infer is not None:
        if known == 0 or total % known:
            raise ValueError("Reshape inferred dimension is not integral")
        target[infer] = total // known
    elif math.prod(target) != total:
        raise ValueError("Reshape target element count does not match input")
    return tuple(target)


def op_reshape(inputs, attrs):
    x = inputs[0]
    shape = resolve_reshape_shape(x.shape, to_host_ints(inputs[1]), int(attrs.get("allowzero", 0)))
    if attrs.get("_planned_output") is None:
        return x.reshape(shape)
    return copy_into(x.reshape(shape), _planned(attrs, shape, x.dtype))


def transpose(x: DeviceArray, perm: Sequence[int], attrs, out_shape: Optional[Sequence[int]] = None) -> DeviceArray:
    if sorted(perm) != list(range(x.ndim)):
        raise ValueError("Transpose perm must contain every axis exactly once")
    src = dense_strides(x.shape)
    tshape = tuple(x.shape[p] for p in perm)
    out = _planned(attrs, tshape if out_shape is None else out_shape, x.dtype)
    strided_copy(x, out, tshape, [src[p] for p in perm])
    return out


def op_transpose(inputs, attrs):
    x = inputs[0]
    perm = attrs.get("perm")
    perm = list(range(x.ndim - 1, -1, -1)) if perm is None else [int(p) for p in perm]
    return transpose(x, perm, attrs)


def softmax(x: DeviceArray, axis: int, attrs, out_dtype=None) -> DeviceArray:
    axis = axis + x.ndim if axis < 0 else axis
    if not 0 <= axis < x.ndim:
        raise ValueError(f"Softmax axis {axis} is invalid for rank {x.ndim}")
    out = _planned(attrs, x.shape, x.dtype if out_dtype is None else out_dtype)
    a = _lib.SoftmaxArgs()
    a.in_, a.out = x.ptr, out.ptr
    a.outer, a.axis, a.inner = math.prod(x.shape[:axis]), x.shape[axis], math.prod(x.shape[axis + 1:])
    a.in_dtype, a.out_dtype = x.code, out.code
    if x.size:
        _lib.launch(a, current_stream())
    return out


def op_softmax(inputs, attrs):
    return softmax(inputs[0], int(attrs.get("axis", -1)), attrs)


# ---------------------------------------------------------------- Conv (NCHW contract)
def conv_geometry(x_shape, w_shape, attrs):
    """(kh, kw, sh, sw, dh, dw, pads[4], ho, wo) with ONNX auto_pad (E:309-374)."""
    n, c, h, w = (int(v) for v in x_shape)
    ks = attrs.get("kernel_shape") or [w_shape[-2], w_shape[-1]]
    kh, kw = int(ks[0]), int(ks[-1]) if len(ks) > 1 else int(ks[0])
    s = list(attrs.get("strides", [1, 1]))
    d = list(attrs.get("dilations", [1, 1]))
    if len(s) != 2 or len(d) != 2:
        raise ValueError("Conv strides/dilations must contain two values")
    sh, sw, dh, dw = int(s[0]), int(s[1]), int(d[0]), int(d[1])
    if min(kh, kw, sh, sw, dh, dw) <= 0:
        raise ValueError("Conv kernel, stride, dilation, and group values must be positive")
    eh, ew = dh * (kh - 1) + 1, dw * (kw - 1) + 1
    auto = attrs.get("auto_pad", "NOTSET")
    auto = (auto.decode() if isinstance(auto, bytes) else str(auto)).upper()
    if auto not in ("NOTSET", "VALID", "SAME_UPPER", "SAME_LOWER"):
        raise ValueError(f"Unsupported Conv auto_pad value: {auto}")
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        oh, ow = math.ceil(h / sh), math.ceil(w / sw)
        th, tw = max((oh - 1) * sh + eh - h, 0), max((ow - 1) * sw + ew - w, 0)
        pt, pl = (th // 2, tw // 2) if auto == "SAME_UPPER" else ((th + 1) // 2, (tw + 1) // 2)
        pads = [pt, pl, th - pt, tw - pl]
    elif auto == "VALID":
        pads = [0, 0, 0, 0]
    else:
        pads = [int(p) for p in attrs.get("pads", [0, 0, 0, 0])]
        if len(pads) != 4 or min(pads) < 0:
            raise ValueError("Conv pads must contain four non-negative values")
    ho = (h + pads[0] + pads[2] - eh) // sh + 1
    wo = (w + pads[1] + pads[3] - ew) // sw + 1
    if ho <= 0 or wo <= 0:
        raise ValueError("Conv attributes produce a non-positive output dimension")
    return kh, kw, sh, sw, dh, dw, pads, ho, wo


def pack_conv_weight(w: DeviceArray, c_pack: int, kw_pack: int, k_stride: int, out_dtype=np.float32,
                     out: Optional[DeviceArray] = None) -> DeviceArray:
    o, c, kh, kw = w.shape
    out = DeviceArray.empty((o, k_stride), out_dtype) if out is None else out
    a = _lib.PackArgs()
    a.w, a.out, a.o, a.c, a.kh, a.kw = w.ptr, out.ptr, o, c, kh, kw
    a.c_pack, a.kw_pack, a.k_stride, a.in_dtype, a.out_dtype = c_pack, kw_pack, k_stride, w.code, out.code
    _lib.launch(a, current_stream())
    return out


def to_nhwc(x: DeviceArray, c_pad: int, out_dtype=np.float32, out: Optional[DeviceArray] = None) -> DeviceArray:
    n, c, h, w = x.shape
    out = DeviceArray.empty((n, h, w, c_pad), out_dtype) if out is None else out
    a = _lib.LayoutArgs()
    a.in_, a.out, a.n, a.c, a.h, a.w = x.ptr, out.ptr, n, c, h, w
    a.c_pad, a.direction, a.in_dtype, a.out_dtype = c_pad, 0, x.code, out.code
    if x.size:
        _lib.launch(a, current_stream())
    return out


def conv2d_nchw(x: DeviceArray, w: DeviceArray, bias: Optional[DeviceArray], attrs, act: int = 0,
                residual: Optional[DeviceArray] = None) -> DeviceArray:
    """NCHW fp32 Conv as one implicit-GEMM launch over a channels-last copy of x."""
    if x.ndim != 4 or w.ndim != 4:
        raise ValueError("This C3 Conv implementation requires rank-4 NCHW tensors")
    group = int(attrs.get("group", 1))
    n, c, h, wd = x.shape
    o = w.shape[0]
    kh, kw, sh, sw, dh, dw, pads, ho, wo = conv_geometry(x.shape, w.shape, attrs)
    if tuple(w.shape[-2:]) != (kh, kw):
        raise ValueError(f"Conv kernel_shape {(kh, kw)} does not match weights {w.shape[-2:]}")
    if c % group or o % group or w.shape[1] != c // group:
        raise ValueError("Conv group is incompatible with input/output channels")
    if bias is not None and (bias.ndim != 1 or bias.shape[0] != o):
        raise ValueError("Conv bias must be one-dimensional with one value per output channel")
    out = _planned(attrs, (n, o, ho, wo))
    cg, og = c // group, o // group
    for g in range(group):
        xg = x if group == 1 else _channel_slice(x, g * cg, cg)
        wg = w if group == 1 else w.ravel().flat(g * og * w.size // o, (g + 1) * og * w.size // o).reshape(
            og, cg, kh, kw)
        c_pad = (cg + 3) // 4 * 4
        xs = to_nhwc(xg, c_pad)
        k = kh * kw * c_pad
        wp = pack_conv_weight(wg, c_pad, kw, k)
        og_out = out if group == 1 else DeviceArray.empty((n, og, ho, wo), np.float32)
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xs.ptr, wp.ptr, og_out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, cg, h, wd, c_pad, c_pad, og
        a.kh, a.kw, a.sh, a.sw = kh, kw, sh, sw
        a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = pads[0], pads[1], dh, dw, ho, wo
        a.out_layout, a.in_dtype, a.out_dtype = 0, _lib.F32, _lib.F32
        bg = None if bias is None else (bias if group == 1 else bias.flat(g * og, (g + 1) * og))
        rg = residual if group == 1 else None
        a.epi = epilogue(bias=bg, bias_mode=2 if bg is not None else 0, act=act if group == 1 else 0,
                         residual=rg)
        if n:
            _lib.launch(a, current_stream())
        if group > 1:
            _copy_channels(og_out, out, g * og)
    if group > 1 and (act or residual is not None):
        prog = []
        ins = [out]
        if residual is not None:
            ins.append(residual)
            prog.append((_lib.EW_ADD, 0, 1, 0.0))
        if act:
            prog.append((_lib.EW_RELU, len(ins) + len(prog) - 1 if prog else 0, 0, 0.0))
        run_ew(ins, prog, {"_planned_output": out})
    return out


def _channel_slice(x: DeviceArray, c0: int, cn: int) -> DeviceArray:
    n, c, h, w = x.shape
    out = DeviceArray.empty((n, cn, h, w), x.dtype)
    strided_copy(x, out, (n, cn, h, w), [c * h * w, h * w, w, 1], offset=c0 * h * w)
    return out


def _copy_channels(src: DeviceArray, dst: DeviceArray, c0: int) -> None:
    n, cn, h, w = src.shape
    c = dst.shape[1]
    for i in range(n):
        copy_into(src.ravel().flat(i * cn * h * w, (i + 1) * cn * h * w),
                  dst.ravel().flat((i * c + c0) * h * w, (i * c + c0 + cn) * h * w))


def op_conv(inputs, attrs):
    return conv2d_nchw(inputs[0], inputs[1], inputs[2] if len(inputs) >= 3 else None, attrs)


def op_batchnorm(inputs, attrs):
    x = inputs[0]
    out = _planned(attrs, x.shape)
    a = _lib.BatchNormArgs()
    a.x, a.scale, a.bias, a.mean, a.var, a.out = x.ptr, inputs[1].ptr, inputs[2].ptr, inputs[3].ptr, inputs[4].ptr, out.ptr
    a.n, a.c, a.hw = x.shape[0], x.shape[1], math.prod(x.shape[2:])
    a.epsilon = float(attrs.get("epsilon", 1e-5))
    if x.size:
        _lib.launch(a, current_stream())
    return out


def op_maxpool(inputs, attrs):
    x = inputs[0]
    if x.ndim != 4:
        raise ValueError("MaxPool requires rank-4 NCHW input")
    if int(attrs.get("ceil_mode", 0)):
        raise NotImplementedError("MaxPool ceil_mode=1 is not supported")
    kh, kw, sh, sw, dh, dw, pads, ho, wo = conv_geometry(x.shape, (0, 0) + tuple(attrs["kernel_shape"]), attrs)
    out = _planned(attrs, (x.shape[0], x.shape[1], ho, wo), x.dtype)
    a = _lib.PoolArgs()
    a.x, a.out = x.ptr, out.ptr
    a.n, a.c, a.h, a.w = x.shape
    a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = kh, kw, sh, sw, pads[0], pads[1], dh, dw, ho, wo
    a.layout, a.c_stride, a.dtype = 0, x.shape[1], x.code
    _lib.launch(a, current_stream())
    return out


# ---------------------------------------------------------------- W8A8 rows (ONNX)
def _scalar(x: DeviceArray) -> float:
    return float(x.get().reshape(-1)[0])


def quantize(x: DeviceArray, scale: float, zero: int, attrs) -> DeviceArray:
    out = _planned(attrs, x.shape, np.int8)
    a = _lib.QuantizeArgs()
    a.x, a.out, a.count, a.scale, a.zero_point, a.x_dtype = x.ptr, out.ptr, x.size, float(scale), int(zero), x.code
    if x.size:
        _lib.launch(a, current_stream())
    return out


def op_quantize_linear(inputs, attrs):
    zero = int(inputs[2].get().reshape(-1)[0]) if len(inputs) > 2 and inputs[2] is not None else 0
    return quantize(inputs[0], _scalar(inputs[1]), zero, attrs)


def dequantize(q: DeviceArray, scale: float, zero: int, attrs, out_dtype=np.float32) -> DeviceArray:
    out = _planned(attrs, q.shape, out_dtype)
    a = _lib.DequantizeArgs()
    a.q, a.out, a.count, a.scale, a.zero_point, a.out_dtype = q.ptr, out.ptr, q.size, float(scale), int(zero), out.code
    if q.size:
        _lib.launch(a, current_stream())
    return out


def op_dequantize_linear(inputs, attrs):
    zero = int(inputs[2].get().reshape(-1)[0]) if len(inputs) > 2 and inputs[2] is not None else 0
    return dequantize(inputs[0], _scalar(inputs[1]), zero, attrs)


def transpose_2d(x: DeviceArray) -> DeviceArray:
    out = DeviceArray.empty((x.shape[1], x.shape[0]), x.dtype)
    strided_copy(x, out, out.shape, [1, x.shape[1]])
    return out


def qgemm(a_q: DeviceArray, b_packed: DeviceArray, out: DeviceArray, m: int, n: int, k: int, mode: int,
          a_scale: float = 1.0, b_scale: Optional[DeviceArray] = None, y_scale: float = 1.0, y_zero: int = 0,
          epi: Optional[_lib.Epilogue] = None) -> None:
    g = _lib.QGemmArgs()
    g.a, g.b, g.out, g.m, g.n, g.k = a_q.ptr, b_packed.ptr, out.ptr, m, n, k
    g.lda, g.ldb, g.ldo = k, k, n
    g.a_zero = g.b_zero = 0
    g.a_scale, g.y_scale = float(a_scale), float(y_scale)
    g.b_scale = b_scale.ptr if b_scale is not None else None
    g.y_zero, g.mode, g.out_dtype = int(y_zero), int(mode), out.code
    g.epi = epi if epi is not None else epilogue()
    _lib.launch(g, current_stream())


def op_qlinear_matmul(inputs, attrs):
    """ONNX QLinearMatMul: int8 x int8 -> exact int32 -> requantized int8."""
    a, sa, za, b, sb, zb, sy, zy = inputs[:8]
    for z in (za, zb, zy):
        if z is not None and np.any(z.get() != 0):
            raise NotImplementedError("QLinearMatMul with nonzero zero points is not supported")
    if b.ndim != 2:
        raise ValueError("QLinearMatMul requires a rank-2 B")
    k, n = b.shape
    lead = a.shape[:-1]
    m = math.prod(lead)
    bt = transpose_2d(b)  # [n][k] packing for the int8 MFMA B operand
    bscale = sb if sb.size == n else _broadcast_scale(sb, n)
    out = _planned(attrs, lead + (n,), np.int8)
    qgemm(a.reshape(m, k), bt, out.reshape(m, n), m, n, k, mode=1, a_scale=_scalar(sa), b_scale=bscale,
          y_scale=_scalar(sy), y_zero=0)
    return out


def _broadcast_scale(s: DeviceArray, n: int) -> DeviceArray:
    return DeviceArray.from_host(np.full(n, float(s.get().reshape(-1)[0]), np.float32))


def op_argmax(inputs, attrs):
    x = inputs[0]
    axis = int(attrs.get("axis", 0))
    axis = axis + x.ndim if axis < 0 else axis
    if axis != x.ndim - 1:
        raise NotImplementedError("ArgMax is implemented along the last axis")
    if int(attrs.get("select_last_index", 0)):
        raise NotImplementedError("ArgMax select_last_index=1 is not supported")
    rows = x.size // x.shape[-1]
    keep = int(attrs.get("keepdims", 1))
    shape = x.shape[:-1] + ((1,) if keep else ())
    out = _planned(attrs, shape, np.int64)
    a = _lib.ArgmaxArgs()
    a.in_, a.out, a.rows, a.cols, a.in_dtype = x.ptr, out.ptr, rows, x.shape[-1], x.code
    if rows:
        _lib.launch(a, current_stream())
    return out


OP_DISPATCH: Dict[str, Any] = {
    "Add": op_add, "Constant": op_constant, "Conv": op_conv, "Div": op_div, "Erf": op_erf,
    "Flatten": op_flatten, "Gather": op_gather, "Gemm": op_gemm, "GlobalAveragePool": op_global_average_pool,
    "LayerNormalization": op_layer_normalization, "MatMul": op_matmul, "Mul": op_mul, "Relu": op_relu,
    "Reshape": op_reshape, "Softmax": op_softmax, "Split": op_split, "Sqrt": op_sqrt, "Sub": op_sub,
    "Transpose": op_transpose, "Exp": op_exp,
    # Rows the reference engine lacks.
    "BatchNormalization": op_batchnorm, "MaxPool": op_maxpool, "QuantizeLinear": op_quantize_linear,
    "QLinearMatMul": op_qlinear_matmul, "DequantizeLinear": op_dequantize_linear, "ArgMax": op_argmax,
}


# ---------------------------------------------------------------- fused ops (E:722-1445)
def op_fused_matmul_bias(inputs, attrs):
    return _execute_gemm_epilogue(inputs, attrs, matmul_semantics=True)


def op_fused_gemm_epilogue(inputs, attrs):
    return _execute_gemm_epilogue(inputs, attrs, matmul_semantics=False)


def op_fused_conv_batchnorm(inputs, attrs):
    if len(inputs) < 2:
        raise ValueError("FusedConv2dBatchNorm requires at least X, W inputs")
    if attrs.get("bn_folded"):
        return op_conv(inputs, attrs)
    off = int(attrs.get("bn_parameter_offset", len(inputs)))
    conv = op_conv(inputs[:off], {k: v for k, v in attrs.items() if k != "_planned_output"})
    if len(inputs) < off + 4:
        raise ValueError("FusedConv2dBatchNorm is missing scale/bias/mean/variance")
    return op_batchnorm([conv] + list(inputs[off:off + 4]), {**attrs, "epsilon": attrs.get("bn_epsilon", 1e-5)})


def _fused_conv_epilogue(inputs, attrs, has_residual: bool):
    if len(inputs) < 2:
        raise ValueError("Fused Conv requires X and W inputs")
    ri = int(attrs.get("_residual_input_index", len(inputs)))
    if has_residual and not 0 <= ri < len(inputs):
        raise ValueError("Fused Conv residual input index is invalid")
    if attrs.get("_activation") != "Relu":
        raise ValueError("Fused Conv epilogue currently requires Relu")
    conv_in = list(inputs[:ri]) if has_residual else list(inputs)
    residual = inputs[ri] if has_residual else None
    return conv2d_nchw(conv_in[0], conv_in[1], conv_in[2] if len(conv_in) > 2 else None, attrs, act=1,
                       residual=residual)


def op_fused_conv_activation(inputs, attrs):
    return _fused_conv_epilogue(inputs, attrs, False)


def op_fused_conv_residual_activation(inputs, attrs):
    return _fused_conv_epilogue(inputs, attrs, True)


def compile_ew_program(ops: Sequence[Dict[str, Any]], n_inputs: int):
    """`_ops` (c33/fusion.py:609-622) -> register program for c3h_ew."""
    if not ops:
        raise ValueError("FusedEWChain has no elementwise program")
    values: Dict[str, int] = {}
    program = []
    for i, entry in enumerate(ops):
        regs = []
        for ref in entry.get("inputs", []):
            if isinstance(ref, int) and 0 <= ref < n_inputs:
                regs.append(ref)
            elif isinstance(ref, str) and ref in values:
                regs.append(values[ref])
            else:
                raise ValueError(f"FusedEWChain cannot resolve operand {ref!r}")
        op = entry.get("op", "")
        if op in _EW_BINARY:
            if len(regs) != 2:
                raise ValueError(f"FusedEWChain {op} expects 2 operands")
            program.append((_EW_BINARY[op], regs[0], regs[1], 0.0))
        elif op in _EW_UNARY_CHAIN:
            if len(regs) != 1:
                raise ValueError(f"FusedEWChain {op} expects 1 operands")
            program.append((_EW_UNARY_CHAIN[op], regs[0], regs[0], 0.0))
        else:
            raise ValueError(f"Unknown op in FusedEWChain: {op}")
        if entry.get("output"):
            values[entry["output"]] = n_inputs + i
    return program


def op_fused_ew_chain(inputs, attrs):
    return run_ew(list(inputs), compile_ew_program(attrs.get("_ops", []), len(inputs)), attrs)


def op_fused_softmax_dropout(inputs, attrs):
    return softmax(inputs[0], int(attrs.get("axis", -1)), attrs)


def op_fused_residual_norm(inputs, attrs):
    if len(inputs) < 3 or inputs[2] is None:
        raise ValueError("FusedResidualNorm requires x, residual and a LayerNorm scale")
    if inputs[0].shape != inputs[1].shape:
        raise ValueError("FusedResidualNorm requires equal residual input shapes")
    return layer_norm(inputs[0], inputs[2], inputs[3] if len(inputs) > 3 else None, int(attrs.get("axis", -1)),
                      float(attrs.get("epsilon", 1e-5)), attrs, residual=inputs[1])


def op_fused_layer_normalization(inputs, attrs):
    if len(inputs) < 2 or inputs[1] is None:
        raise ValueError("Fused LayerNormalization requires X and Scale")
    return layer_norm(inputs[0], inputs[1], inputs[2] if len(inputs) > 2 else None, int(attrs.get("axis", -1)),
                      float(attrs.get("epsilon", 1e-5)), attrs)


def op_fused_attention_scores(inputs, attrs):
    if len(inputs) != 4:
        raise ValueError("FusedAttentionScores requires Q, K, divisor, and mask")
    q, kt, div, mask = inputs
    if q.ndim != 4 or kt.ndim != 4:
        raise ValueError("FusedAttentionScores requires rank-4 MatMul inputs")
    if div.size != 1:
        raise ValueError("FusedAttentionScores divisor must be scalar")
    q0, q1, rows, inner = q.shape
    k0, k1, kinner, cols = kt.shape
    if inner != kinner:
        raise ValueError("FusedAttentionScores MatMul inner dimensions differ")
    out0, out1 = max(q0, k0), max(q1, k1)
    mshape = [1] * (4 - mask.ndim) + list(mask.shape)
    out = _planned(attrs, (out0, out1, rows, cols))
    a = _lib.AttnScoresArgs()
    a.q, a.kt, a.divisor, a.mask, a.out = q.ptr, kt.ptr, div.ptr, mask.ptr, out.ptr
    a.q0, a.q1, a.k0, a.k1, a.rows, a.cols, a.inner = q0, q1, k0, k1, rows, cols, inner
    a.m0, a.m1, a.m2, a.m3 = mshape
    a.in_dtype = q.code
    _lib.launch(a, current_stream())
    return out


def op_fused_transpose_reshape(inputs, attrs):
    x = inputs[0]
    if not 1 <= x.ndim <= 4:
        raise ValueError("FusedTransposeReshape supports ranks one through four")
    perm = [int(p) for p in attrs.get("perm", range(x.ndim - 1, -1, -1))]
    tshape = tuple(x.shape[p] for p in perm)
    shape = resolve_reshape_shape(tshape, to_host_ints(inputs[1]), int(attrs.get("allowzero", 0)))
    return transpose(x, perm, attrs, out_shape=shape)


def op_fused_residual_relu(inputs, attrs):
    return run_ew([inputs[0], inputs[1]], [(_lib.EW_ADD, 0, 1, 0.0), (_lib.EW_RELU, 2, 2, 0.0)], attrs)


OP_DISPATCH.update({
    "FusedMatMulBias": op_fused_matmul_bias,
    "FusedGemmEpilogue": op_fused_gemm_epilogue,
    "FusedConv2dBatchNorm": op_fused_conv_batchnorm,
    "FusedConvActivation": op_fused_conv_activation,
    "FusedConvResidualActivation": op_fused_conv_residual_activation,
    "FusedAttentionScores": op_fused_attention_scores,
    "FusedEWChain": op_fused_ew_chain,
    "FusedLayerNormalization": op_fused_layer_normalization,
    "FusedSoftmaxDropout": op_fused_softmax_dropout,
    "FusedResidualNorm": op_fused_residual_norm,
    "FusedTransposeReshape": op_fused_transpose_reshape,
})


def execute_op(op_type: str, inputs: List[DeviceArray], attrs: Dict[str, Any]) -> Any:
    impl = OP_DISPATCH.get(op_type)
    if impl is None:
        raise ValueError(f"Unknown operator type: {op_type}")
    return impl(inputs, attrs)
