"""CPU oracle of the C3.2 kernel registry and the C3.5 fused ops (NumPy).

TEST INFRASTRUCTURE ONLY.  Only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s CPU-baseline leg may import this package, and only as the
checker; the product path (hackathon_amd) never imports it.

Each kernel restates one reference registry body
(c32/kernel_registry.py, "R") or engine op (c35/engine.py, "E") with the same
signature `fn(inputs, outputs, params, tuning)`, NumPy arrays in place of CuPy
arrays.  Results are written like the reference's `_write_result`
(R:84-102): into the front of the flat output buffer, and `outputs[i]` is
replaced by the correctly shaped view.  Unlike the reference, every step
computes fp32 with NumPy BLAS; fp32 parity with the HIP path is therefore a
tolerance check, not a bitwise one.

Functions the reference lacks (MaxPool, Quantize/QLinearMatMul/Dequantize,
ArgMax) restate the ONNX opset-17 definitions.
"""

from __future__ import annotations

import math
from typing import Any, Callable, Dict, List, Optional

import numpy as np
from scipy import special as _special

F32 = np.float32
_REGISTRY: Dict[str, Callable[..., None]] = {}


def register(*names: str):
    def deco(fn):
        for n in names:
            _REGISTRY[n] = fn
        return fn
    return deco


def lookup(name: str) -> Callable[..., None]:
    """R:42-67 name resolution: verbatim, +_f32, -_f32, _fp32 -> _f32."""
    if name in _REGISTRY:
        return _REGISTRY[name]
    if f"{name}_f32" in _REGISTRY:
        return _REGISTRY[f"{name}_f32"]
    if name.endswith("_f32") and name[:-4] in _REGISTRY:
        return _REGISTRY[name[:-4]]
    if name.endswith("_fp32"):
        bare = name[:-5]
        for cand in (f"{bare}_f32", bare):
            if cand in _REGISTRY:
                return _REGISTRY[cand]
    raise RuntimeError(f"Unknown kernel: {name!r}.  Registered kernels: {sorted(_REGISTRY)}")


def _write(output: np.ndarray, result: np.ndarray) -> np.ndarray:
    """R:84-102: copy into the front of the capacity view, return the shaped view."""
    result = np.asarray(result)
    need = int(result.size)
    flat = output.reshape(-1)
    if flat.size < need:
        raise ValueError(f"Output arena too small: need {need} elements, have {flat.size}")
    dest = flat[:need].reshape(result.shape)
    dest[...] = result
    return dest


def erf_as(x: np.ndarray) -> np.ndarray:
    """Abramowitz & Stegun 7.1.26 in float32 arithmetic (R:180-193, E:201-223)."""
    x = np.asarray(x, F32)
    sign = np.sign(x)
    ax = np.abs(x)
    t = F32(1.0) / (F32(1.0) + F32(0.3275911) * ax)
    t2 = t * t
    t3 = t2 * t
    t4 = t3 * t
    t5 = t4 * t
    c = np.asarray([0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429], F32)
    poly = c[0] * t + c[1] * t2 + c[2] * t3 + c[3] * t4 + c[4] * t5
    return (sign * (F32(1.0) - poly * np.exp(-ax * ax))).astype(F32)


def erf_exact(x: np.ndarray) -> np.ndarray:
    """erf in float64, rounded to float32 (fused-chain erf, E:965)."""
    return _special.erf(np.asarray(x, np.float64)).astype(F32)


# -- elementwise -------------------------------------------------------------------------
@register("add", "add_f32")
def kernel_add(inputs, outputs, params, tuning):
    if "epsilon" in params and len(inputs) == 1:
        outputs[0] = _write(outputs[0], np.add(inputs[0], F32(params["epsilon"]), dtype=F32))
    else:
        outputs[0] = _write(outputs[0], np.add(inputs[0], inputs[1], dtype=F32))


@register("mul", "mul_f32")
def kernel_mul(inputs, outputs, params, tuning):
    # The reference writes through out= into the flat capacity view (R:214),
    # which only works for flat-compatible shapes; here the broadcast result
    # is written like every other step.
    outputs[0] = _write(outputs[0], np.multiply(inputs[0], inputs[1], dtype=F32))


@register("div", "div_f32")
def kernel_div(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.divide(inputs[0], inputs[1], dtype=F32))


@register("sub", "sub_f32")
def kernel_sub(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.subtract(inputs[0], inputs[1], dtype=F32))


@register("relu_f32")
def kernel_relu(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.maximum(inputs[0], F32(0)))


@register("erf_f32")
def kernel_erf(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], erf_as(inputs[0]))


@register("exp", "exp_f32")
def kernel_exp(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.exp(inputs[0], dtype=F32))


@register("sqrt", "sqrt_f32")
def kernel_sqrt(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.sqrt(inputs[0], dtype=F32))


@register("reciprocal", "reciprocal_f32")
def kernel_reciprocal(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.reciprocal(np.asarray(inputs[0], F32)))


# -- reductions (R:272-311) --------------------------------------------------------------
def reduction_axes(params: Dict[str, Any], ndim: int):
    axes, axis = params.get("axes"), params.get("axis")
    keepdims = bool(params.get("keepdims", False))
    if axes is not None:
        if isinstance(axes, (list, tuple)):
            return tuple(int(a) % ndim for a in axes), keepdims
        return (int(axes) % ndim,), keepdims
    if axis is not None:
        return (int(axis) % ndim,), keepdims
    return tuple(range(ndim)), keepdims


@register("reduce_max", "reduce_max_f32")
def kernel_reduce_max(inputs, outputs, params, tuning):
    axes, keep = reduction_axes(params, inputs[0].ndim)
    outputs[0] = _write(outputs[0], np.max(inputs[0], axis=axes, keepdims=keep))


@register("reduce_sum", "reduce_sum_f32")
def kernel_reduce_sum(inputs, outputs, params, tuning):
    axes, keep = reduction_axes(params, inputs[0].ndim)
    outputs[0] = _write(outputs[0], np.sum(inputs[0], axis=axes, keepdims=keep, dtype=F32))


@register("reduce_mean", "reduce_mean_f32")
def kernel_reduce_mean(inputs, outputs, params, tuning):
    axes, keep = reduction_axes(params, inputs[0].ndim)
    outputs[0] = _write(outputs[0], np.mean(inputs[0], axis=axes, keepdims=keep, dtype=F32))


# -- matmul / conv lowering (R:318-453) ------------------------------------------------------
@register("matmul_f32")
def kernel_matmul(inputs, outputs, params, tuning):
    a = np.asarray(inputs[0], F32)
    b = np.asarray(inputs[1], F32)
    ta, tb = int(params.get("transA", 0)), int(params.get("transB", 0))
    alpha = float(params.get("alpha", 1.0))
    if params.get("lowering_kind", "matmul") == "conv_contract":
        b2 = b.reshape(b.shape[0], -1).T if b.ndim == 4 else b
        if ta:
            a = a.T
        if tb:
            b2 = b2.T
        result = a @ b2
    else:
        if ta:
            a = a.T
        if tb:
            b = b.T
        result = np.dot(a, b) if a.ndim == 2 and b.ndim == 2 else np.matmul(a, b)
    if alpha != 1.0:
        result = result * F32(alpha)
    outputs[0] = _write(outputs[0], result.astype(F32, copy=False))


def reshape_conv_output(result: np.ndarray, params: Dict[str, Any]) -> np.ndarray:
    """[N*Ho*Wo, O] (rows n, ho, wo) -> NCHW (R:105-175)."""
    if result.ndim != 2:
        return result
    m, o = result.shape
    n = params.get("_batch_size")
    if not n or m % int(n):
        return result
    n = int(n)
    hw = m // n

    def nchw(h, w):
        return result.reshape(n, h, w, o).transpose(0, 3, 1, 2)

    s = params.get("strides", [1, 1])
    sh, sw = int(s[0]), int(s[-1])
    pt, pl, pb, pr = [int(p) for p in params.get("pads", [0, 0, 0, 0])]
    d = params.get("dilations", [1, 1])
    dh, dw = int(d[0]), int(d[-1])
    ks = params.get("kernel_shape", [3, 3])
    kh, kw = int(ks[0]), int(ks[-1])
    out_sp = params.get("_output_spatial")
    if out_sp and len(out_sp) == 2 and int(out_sp[0]) > 0 and int(out_sp[0]) * int(out_sp[1]) == hw:
        return nchw(int(out_sp[0]), int(out_sp[1]))
    in_sp = params.get("_input_spatial")
    if in_sp and len(in_sp) == 2:
        ho = (int(in_sp[0]) + pt + pb - dh * (kh - 1) - 1) // sh + 1
        wo = (int(in_sp[1]) + pl + pr - dw * (kw - 1) - 1) // sw + 1
        if ho > 0 and wo > 0 and ho * wo == hw:
            return nchw(ho, wo)
    h = math.isqrt(hw)
    while h > 0:
        if hw % h == 0:
            w = hw // h
            if (h - 1) * sh - pt - pb + dh * (kh - 1) + 1 > 0 and (w - 1) * sw - pl - pr + dw * (kw - 1) + 1 > 0:
                return nchw(h, w)
        h -= 1
    return result


@register("conv_reshape_f32")
def kernel_conv_reshape(inputs, outputs, params, tuning):
    r = inputs[0]
    if r.ndim == 2:
        r = reshape_conv_output(r, params)
    outputs[0] = _write(outputs[0], np.asarray(r, F32))


@register("add_bias_f32")
def kernel_add_bias(inputs, outputs, params, tuning):
    data, bias = inputs[0], inputs[1]
    beta = float(params.get("beta", 1.0))
    axis = int(params.get("bias_axis", -1))
    axis = axis + data.ndim if axis < 0 else axis
    shape = [1] * data.ndim
    shape[axis] = int(bias.size)
    outputs[0] = _write(outputs[0], (data + bias.reshape(shape) * F32(beta)).astype(F32))


def conv_geometry(x_shape, params):
    ks = params.get("kernel_shape", [3, 3])
    kh, kw = int(ks[0]), int(ks[-1]) if len(ks) > 1 else int(ks[0])
    s = list(params.get("strides", [1, 1]))
    sh, sw = int(s[0]), int(s[-1])
    d = list(params.get("dilations", [1, 1]))
    dh, dw = int(d[0]), int(d[-1])
    pt, pl, pb, pr = [int(p) for p in params.get("pads", [0, 0, 0, 0])]
    n, c, h, w = x_shape
    ho = (h + pt + pb - (dh * (kh - 1) + 1)) // sh + 1
    wo = (w + pl + pr - (dw * (kw - 1) + 1)) // sw + 1
    return kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, ho, wo


def im2col(x: np.ndarray, params: Dict[str, Any]) -> np.ndarray:
    """[N*Ho*Wo, C*kh*kw], rows (n, ho, wo), columns (c, kh, kw) (R:399-453)."""
    x = np.asarray(x, F32)
    if x.ndim != 4:
        raise ValueError("im2col requires rank-4 NCHW input")
    kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, ho, wo = conv_geometry(x.shape, params)
    n, c = x.shape[:2]
    xp = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    cols = np.empty((n, ho, wo, c, kh, kw), F32)
    for i in range(kh):
        for j in range(kw):
            patch = xp[:, :, i * dh:i * dh + sh * (ho - 1) + 1:sh, j * dw:j * dw + sw * (wo - 1) + 1:sw]
            cols[:, :, :, :, i, j] = patch.transpose(0, 2, 3, 1)
    return cols.reshape(n * ho * wo, c * kh * kw)


@register("im2col_f32")
def kernel_im2col(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], im2col(inputs[0], params))


def conv2d(x: np.ndarray, w: np.ndarray, params: Dict[str, Any], bias: Optional[np.ndarray] = None) -> np.ndarray:
    """NCHW conv via im2col + contraction (E:288-440), groups supported."""
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    group = int(params.get("group", 1))
    n, c = x.shape[:2]
    o = w.shape[0]
    kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, ho, wo = conv_geometry(x.shape, params)
    outs = []
    cg, og = c // group, o // group
    for g in range(group):
        cols = im2col(x[:, g * cg:(g + 1) * cg], params)
        wg = w[g * og:(g + 1) * og].reshape(og, -1)
        outs.append((cols @ wg.T).reshape(n, ho, wo, og).transpose(0, 3, 1, 2))
    out = np.concatenate(outs, axis=1) if group > 1 else outs[0]
    if bias is not None:
        out = out + np.asarray(bias, F32).reshape(1, o, 1, 1)
    return np.ascontiguousarray(out, F32)


@register("winograd_forward_f32")
def kernel_winograd_forward(inputs, outputs, params, tuning):
    """Conv semantics for the 3x3 s1 step (the reference's body cannot run padded convs, R:540-566)."""
    outputs[0] = _write(outputs[0], conv2d(inputs[0], inputs[1], params))


@register("batchnorm_f32")
def kernel_batchnorm(inputs, outputs, params, tuning):
    x = np.asarray(inputs[0], F32)
    shp = (1, -1) + (1,) * (x.ndim - 2)
    scale, bias, mean, var = (np.asarray(v, F32).reshape(shp) for v in inputs[1:5])
    eps = F32(params.get("epsilon", 1e-5))
    outputs[0] = _write(outputs[0], ((x - mean) / np.sqrt(var + eps) * scale + bias).astype(F32))


# -- fused ops (E:722-1445) ---------------------------------------------------------------
def gemm_epilogue(inputs: List[np.ndarray], attrs: Dict[str, Any], matmul_semantics: bool) -> np.ndarray:
    a = np.asarray(inputs[0], F32)
    b = np.asarray(inputs[1], F32)
    fa = attrs.get("_flatten_axis")
    if fa is not None:
        ax = int(fa) + (a.ndim if int(fa) < 0 else 0)
        a = a.reshape(math.prod(a.shape[:ax]), math.prod(a.shape[ax:]))
    lead = ()
    if matmul_semantics:
        lead = a.shape[:-1]
        a = a.reshape(-1, a.shape[-1])
        ta = tb = 0
    else:
        ta, tb = int(attrs.get("transA", 0)), int(attrs.get("transB", 0))
    a2 = a.T if ta else a
    b2 = b.T if tb else b
    acc = a2 @ b2
    v = F32(attrs.get("alpha", 1.0)) * acc
    if len(inputs) >= 3 and inputs[2] is not None:
        c = np.asarray(inputs[2], F32)
        cs = list(c.shape)
        while len(cs) > 2 and cs[0] == 1:
            cs.pop(0)
        c = c.reshape(cs) if cs else c.reshape(1, 1)
        if c.ndim == 1:
            c = c.reshape(1, -1)
        v = v + F32(attrs.get("beta", 1.0)) * c
    if attrs.get("_activation") == "Relu":
        v = np.maximum(v, F32(0))
    v = v.astype(F32)
    return v.reshape(lead + (v.shape[-1],)) if matmul_semantics else v


@register("fused_matmul_bias_f32")
def kernel_fused_matmul_bias(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], gemm_epilogue(inputs, params, True))


@register("fused_gemm_epilogue_f32")
def kernel_fused_gemm_epilogue(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], gemm_epilogue(inputs, params, False))


EW_UNARY = {"Relu": lambda a: np.maximum(a, F32(0)), "Erf": erf_exact, "Sqrt": np.sqrt, "Exp": np.exp}
EW_BINARY = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}


def ew_chain(inputs: List[np.ndarray], attrs: Dict[str, Any]) -> np.ndarray:
    """Interpret the `_ops` program (c33/fusion.py:609-622, E:948-1013)."""
    ops = attrs.get("_ops", [])
    if not ops:
        raise ValueError("FusedEWChain has no elementwise program")
    values: Dict[str, np.ndarray] = {}
    result = None
    for entry in ops:
        args = []
        for ref in entry.get("inputs", []):
            if isinstance(ref, int) and 0 <= ref < len(inputs):
                args.append(np.asarray(inputs[ref], F32))
            elif isinstance(ref, str) and ref in values:
                args.append(values[ref])
            else:
                raise ValueError(f"FusedEWChain cannot resolve operand {ref!r}")
        op = entry.get("op", "")
        if op in EW_UNARY:
            result = EW_UNARY[op](args[0]).astype(F32)
        elif op in EW_BINARY:
            result = EW_BINARY[op](args[0], args[1]).astype(F32)
        else:
            raise ValueError(f"Unknown op in FusedEWChain: {op}")
        if entry.get("output"):
            values[entry["output"]] = result
    return result


@register("fused_ew_f32")
def kernel_fused_ew(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], ew_chain(inputs, params))


def softmax(x: np.ndarray, axis: int) -> np.ndarray:
    x = np.asarray(x, F32)
    m = x.max(axis=axis, keepdims=True)
    e = np.exp(x - m)
    return (e / e.sum(axis=axis, keepdims=True)).astype(F32)


@register("fused_softmax_f32")
def kernel_fused_softmax(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], softmax(inputs[0], int(params.get("axis", -1))))


def layer_norm(x, scale, bias, axis: int, eps: float):
    x = np.asarray(x, F32)
    axis = axis + x.ndim if axis < 0 else axis
    axes = tuple(range(axis, x.ndim))
    mean = x.mean(axis=axes, keepdims=True, dtype=F32)
    centered = x - mean
    var = np.mean(centered * centered, axis=axes, keepdims=True, dtype=F32)
    inv = F32(1.0) / np.sqrt(var + F32(eps))
    y = centered * inv * np.asarray(scale, F32).reshape(x.shape[axis:])
    if bias is not None:
        y = y + np.asarray(bias, F32).reshape(x.shape[axis:])
    return y.astype(F32), mean.astype(F32), inv.astype(F32)


@register("fused_residual_norm_f32")
def kernel_fused_residual_norm(inputs, outputs, params, tuning):
    x = np.asarray(inputs[0], F32) + np.asarray(inputs[1], F32)
    bias = inputs[3] if len(inputs) > 3 else None
    y, _, _ = layer_norm(x, inputs[2], bias, int(params.get("axis", -1)), float(params.get("epsilon", 1e-5)))
    outputs[0] = _write(outputs[0], y)


@register("fused_layer_norm_f32")
def kernel_fused_layer_norm(inputs, outputs, params, tuning):
    bias = inputs[2] if len(inputs) > 2 else None
    y, _, _ = layer_norm(inputs[0], inputs[1], bias, int(params.get("axis", -1)), float(params.get("epsilon", 1e-5)))
    outputs[0] = _write(outputs[0], y)


def attention_scores(q, kt, divisor, mask) -> np.ndarray:
    s = np.matmul(np.asarray(q, F32), np.asarray(kt, F32)) / np.asarray(divisor, F32).reshape(())
    return softmax(s + np.asarray(mask, F32), -1)


@register("fused_attention_scores_f32")
def kernel_fused_attention_scores(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], attention_scores(*inputs[:4]))


def resolve_reshape(in_shape, shape_value, allowzero: int):
    """ONNX Reshape shape resolution (E:72-107)."""
    raw = [int(v) for v in np.asarray(shape_value).reshape(-1).tolist()]
    target, infer, known = [], None, 1
    for i, d in enumerate(raw):
        if d == 0 and not allowzero:
            d = int(in_shape[i])
        if d == -1:
            infer = i
            target.append(-1)
        else:
            target.append(d)
            known *= d
    total = math.prod(int(v) for v in in_shape)
    if infer is not None:
        target[infer] = total // known
    return tuple(target)


@register("fused_transpose_reshape_f32")
def kernel_fused_transpose_reshape(inputs, outputs, params, tuning):
    x = np.asarray(inputs[0])
    perm = [int(p) for p in params.get("perm", range(x.ndim - 1, -1, -1))]
    t = np.transpose(x, perm)
    outputs[0] = _write(outputs[0], t.reshape(resolve_reshape(t.shape, inputs[1], int(params.get("allowzero", 0)))))


@register("fused_residual_relu_f32")
def kernel_fused_residual_relu(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], np.maximum(np.asarray(inputs[0], F32) + np.asarray(inputs[1], F32), F32(0)))


# -- metadata / data movement (R:669-759) -------------------------------------------------
@register("reshape")
def kernel_reshape(inputs, outputs, params, tuning):
    x = inputs[0]
    if len(inputs) >= 2 and inputs[1] is not None and np.asarray(inputs[1]).size > 0:
        shape = resolve_reshape(x.shape, inputs[1], int(params.get("allowzero", 0)))
    else:
        shape = tuple(params.get("_reshape_shape", x.shape))
    outputs[0] = _write(outputs[0], np.reshape(x, shape))


@register("transpose")
def kernel_transpose(inputs, outputs, params, tuning):
    x = inputs[0]
    perm = params.get("perm")
    perm = list(range(x.ndim - 1, -1, -1)) if perm is None else [int(p) for p in perm]
    outputs[0] = _write(outputs[0], np.transpose(x, perm))


@register("flatten")
def kernel_flatten(inputs, outputs, params, tuning):
    x = inputs[0]
    axis = int(params.get("axis", 1))
    axis = axis + x.ndim if axis < 0 else axis
    outputs[0] = _write(outputs[0], x.reshape(math.prod(x.shape[:axis]), math.prod(x.shape[axis:])))


@register("split")
def kernel_split(inputs, outputs, params, tuning):
    x = inputs[0]
    axis = int(params.get("axis", 0))
    sizes = list(params.get("split", []))
    n_out = int(params.get("_num_outputs", len(outputs)))
    if not sizes:
        if n_out <= 0 or x.shape[axis] % n_out:
            raise ValueError("Split requires equal division")
        sizes = [x.shape[axis] // n_out] * n_out
    bounds = np.cumsum([int(s) for s in sizes[:-1]]).tolist()
    for i, part in enumerate(np.split(x, bounds, axis=axis)):
        if i < len(outputs):
            outputs[i] = _write(outputs[i], part)


@register("gather")
def kernel_gather(inputs, outputs, params, tuning):
    x = inputs[0]
    axis = int(params.get("axis", 0))
    axis = axis + x.ndim if axis < 0 else axis
    outputs[0] = _write(outputs[0], np.take(x, np.asarray(inputs[1], np.int64), axis=axis))


@register("constant")
def kernel_constant(inputs, outputs, params, tuning):
    pass


# -- rows the reference lacks (ONNX opset 17) -------------------------------------------------
def maxpool2d(x: np.ndarray, params: Dict[str, Any]) -> np.ndarray:
    x = np.asarray(x)
    kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, ho, wo = conv_geometry(x.shape, params)
    xp = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)), constant_values=-np.inf)
    out = np.full(x.shape[:2] + (ho, wo), -np.inf, x.dtype)
    for i in range(kh):
        for j in range(kw):
            out = np.maximum(out, xp[:, :, i * dh:i * dh + sh * (ho - 1) + 1:sh, j * dw:j * dw + sw * (wo - 1) + 1:sw])
    return out


@register("maxpool_f32")
def kernel_maxpool(inputs, outputs, params, tuning):
    outputs[0] = _write(outputs[0], maxpool2d(inputs[0], params))


def quantize(x, scale, zero) -> np.ndarray:
    """ONNX QuantizeLinear to int8: saturate(round_half_even(x / scale) + zero)."""
    q = np.rint(np.asarray(x, F32) / F32(np.asarray(scale).reshape(()))) + F32(np.asarray(zero).reshape(()))
    return np.clip(q, -128, 127).astype(np.int8)


def qlinear_matmul_acc(a_q: np.ndarray, a_zero, b_q: np.ndarray, b_zero) -> np.ndarray:
    """Exact int32 accumulators sum_k (a - za)(b - zb) (float64 BLAS is exact below 2**53)."""
    a = a_q.astype(np.float64) - float(np.asarray(a_zero).reshape(()))
    b = b_q.astype(np.float64) - np.asarray(b_zero, np.float64)
    return np.matmul(a, b).astype(np.int64).astype(np.int32)


def requantize(acc: np.ndarray, a_scale, b_scale, y_scale, y_zero) -> np.ndarray:
    """y = saturate(rne(acc * (a_scale*b_scale[n]) / y_scale) + y_zero), fp32 arithmetic."""
    mult = (F32(np.asarray(a_scale).reshape(())) * np.asarray(b_scale, F32)) / F32(np.asarray(y_scale).reshape(()))
    y = np.rint(acc.astype(F32) * mult.astype(F32)) + F32(np.asarray(y_zero).reshape(()))
    return np.clip(y, -128, 127).astype(np.int8)


@register("quantize_linear")
def kernel_quantize_linear(inputs, outputs, params, tuning):
    zero = inputs[2] if len(inputs) > 2 and inputs[2] is not None else 0
    outputs[0] = _write(outputs[0], quantize(inputs[0], inputs[1], zero))


@register("qlinear_matmul")
def kernel_qlinear_matmul(inputs, outputs, params, tuning):
    a, sa, za, b, sb, zb, sy, zy = inputs[:8]
    acc = qlinear_matmul_acc(a, za, b, zb)
    outputs[0] = _write(outputs[0], requantize(acc, sa, sb, sy, zy))


@register("dequantize_linear")
def kernel_dequantize_linear(inputs, outputs, params, tuning):
    zero = inputs[2] if len(inputs) > 2 and inputs[2] is not None else 0
    y = (np.asarray(inputs[0], np.int32) - np.int32(np.asarray(zero).reshape(()))).astype(F32) * \
        F32(np.asarray(inputs[1]).reshape(()))
    outputs[0] = _write(outputs[0], y.astype(F32))


@register("argmax")
def kernel_argmax(inputs, outputs, params, tuning):
    x = np.asarray(inputs[0])
    axis = int(params.get("axis", 0))
    r = np.argmax(x, axis=axis)
    if int(params.get("keepdims", 1)):
        r = np.expand_dims(r, axis)
    outputs[0] = _write(outputs[0], r.astype(np.int64))


def registered() -> List[str]:
    return sorted(_REGISTRY)
