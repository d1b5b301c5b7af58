"""Kernel registry: C3.2 kernel names -> HIP kernel launches (counterpart of
c32/kernel_registry.py).

Same lookup contract as the reference (R:34-81): `register`, `lookup` with
`_f32` / `_fp32` normalization, `is_registered`, `list_registered`, and a
fail-closed RuntimeError for unknown names.  Same kernel signature
(R:6-17):

    fn(inputs: List[DeviceArray | None], outputs: List[DeviceArray],
       params: Dict[str, Any], tuning: Optional[Dict[str, int]]) -> None

`outputs[i]` arrives as a full-capacity arena view; the kernel writes its
result at the front of that view and replaces `outputs[i]` with the shaped
view (R:84-102) - directly from the kernel, without the reference's
temporary + D2D copy.  Every body is a libc3hip.so launch on the current
stream.
"""

from __future__ import annotations

import math
from typing import Any, Callable, Dict, List, Optional

import numpy as np

from .. import _lib
from ..c35 import engine as E
from ..device import DeviceArray, current_stream

KernelFunc = Callable[..., None]
_registry: Dict[str, KernelFunc] = {}


def register(name: str) -> Callable[[KernelFunc], KernelFunc]:
    def decorator(fn: KernelFunc) -> KernelFunc:
        _registry[name] = fn
        return fn
    return decorator


def lookup(name: str) -> KernelFunc:
    if name in _registry:
        return _registry[name]
    if f"{name}_f32" in _registry:
        return _registry[f"{name}_f32"]
    if name.endswith("_f32") and name[:-4] in _registry:
        return _registry[name[:-4]]
    if name.endswith("_fp32"):
        bare = name[:-5]
        if f"{bare}_f32" in _registry:
            return _registry[f"{bare}_f32"]
        if bare in _registry:
            return _registry[bare]
    raise RuntimeError(f"Unknown kernel: {name!r}.  Registered kernels: {sorted(_registry)}")


def is_registered(name: str) -> bool:
    try:
        lookup(name)
        return True
    except RuntimeError:
        return False


def list_registered() -> List[str]:
    return sorted(_registry)


def _out(outputs: List[DeviceArray], i: int = 0) -> Dict[str, Any]:
    return {"_planned_output": outputs[i] if i < len(outputs) else None}


def _regs(*names):
    def deco(fn):
        for n in names:
            register(n)(fn)
        return fn
    return deco


# -- elementwise (R:200-265) -----------------------------------------------------------------
@_regs("add", "add_f32")
def kernel_add(inputs, outputs, params, tuning):
    if "epsilon" in params and len(inputs) == 1:
        outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_ADD_IMM, 0, 0, float(params["epsilon"]))], _out(outputs))
    else:
        outputs[0] = E.run_ew([inputs[0], inputs[1]], [(_lib.EW_ADD, 0, 1, 0.0)], _out(outputs))


@_regs("mul", "mul_f32")
def kernel_mul(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0], inputs[1]], [(_lib.EW_MUL, 0, 1, 0.0)], _out(outputs))


@_regs("div", "div_f32")
def kernel_div(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0], inputs[1]], [(_lib.EW_DIV, 0, 1, 0.0)], _out(outputs))


@_regs("sub", "sub_f32")
def kernel_sub(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0], inputs[1]], [(_lib.EW_SUB, 0, 1, 0.0)], _out(outputs))


@register("relu_f32")
def kernel_relu(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_RELU, 0, 0, 0.0)], _out(outputs))


@register("erf_f32")
def kernel_erf(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_ERF_AS, 0, 0, 0.0)], _out(outputs))


@_regs("exp", "exp_f32")
def kernel_exp(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_EXP, 0, 0, 0.0)], _out(outputs))


@_regs("sqrt", "sqrt_f32")
def kernel_sqrt(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_SQRT, 0, 0, 0.0)], _out(outputs))


@_regs("reciprocal", "reciprocal_f32")
def kernel_reciprocal(inputs, outputs, params, tuning):
    outputs[0] = E.run_ew([inputs[0]], [(_lib.EW_RECIP, 0, 0, 0.0)], _out(outputs))


# -- reductions (R:272-311) ------------------------------------------------------------------------
def _reduction_axes(params: Dict[str, Any], ndim: int):
    axes, axis = params.get("axes"), params.get("axis")
    keep = bool(params.get("keepdims", False))
    if axes is not None:
        if isinstance(axes, (list, tuple)):
            return tuple(int(a) % ndim for a in axes), keep
        return (int(axes) % ndim,), keep
    if axis is not None:
        return (int(axis) % ndim,), keep
    return tuple(range(ndim)), keep


def _reduce(kind: int):
    def fn(inputs, outputs, params, tuning):
        axes, keep = _reduction_axes(params, inputs[0].ndim)
        outputs[0] = E.reduce(inputs[0], axes, keep, kind, _out(outputs))
    return fn


register("reduce_max")(_reduce(0))
register("reduce_max_f32")(_reduce(0))
register("reduce_sum")(_reduce(1))
register("reduce_sum_f32")(_reduce(1))
register("reduce_mean")(_reduce(2))
register("reduce_mean_f32")(_reduce(2))


# -- matmul / conv lowering (R:318-453) -------------------------------------------------------------
@register("matmul_f32")
def kernel_matmul(inputs, outputs, params, tuning):
    a, b = inputs[0], inputs[1]
    ta, tb = int(params.get("transA", 0)), int(params.get("transB", 0))
    alpha = float(params.get("alpha", 1.0))
    lowering = params.get("lowering_kind", "matmul")
    if lowering == "conv_contract" or (a.ndim == 2 and b.ndim in (2, 4)):
        # conv_contract: B = weight [O, C, kh, kw] viewed as [O, CKK] (K-contiguous rows).
        if lowering == "conv_contract" and b.ndim == 4:
            b2 = b.reshape(b.shape[0], -1)
            tb_eff = 1 - tb  # the reference contracts with W.reshape(O,-1).T
        else:
            b2 = b
            tb_eff = tb
        m = a.shape[1] if ta else a.shape[0]
        k = a.shape[0] if ta else a.shape[1]
        n = b2.shape[0] if tb_eff else b2.shape[1]
        kb = b2.shape[1] if tb_eff else b2.shape[0]
        if k != kb:
            raise ValueError(f"matmul inner dimensions differ: {k} and {kb}")
        out = E._planned(_out(outputs), (m, n))
        E.gemm(a, b2, out, m, n, k, lda=a.shape[1], ldb=b2.shape[1], ldo=n, trans_a=ta, trans_b=tb_eff,
               epi=E.epilogue(alpha=alpha))
        outputs[0] = out
        return
    if ta or tb:
        raise NotImplementedError("transA/transB on batched matmul operands")
    outputs[0] = E.op_matmul([a, b], {**_out(outputs), "alpha": alpha})


def conv_output_spatial(m: int, o: int, params: Dict[str, Any]):
    """(N, Ho, Wo) of an NHWO [M, O] contraction (R:105-175), or None."""
    n = params.get("_batch_size")
    if not n or m % int(n):
        return None
    n = int(n)
    hw = m // n
    s = params.get("strides", [1, 1])
    sh, sw = int(s[0]), int(s[-1])
    pt, pl, pb, pr = [int(p) for p in params.get("pads", [0, 0, 0, 0])]
    d = params.get("dilations", [1, 1])
    dh, dw = int(d[0]), int(d[-1])
    ks = params.get("kernel_shape", [3, 3])
    kh, kw = int(ks[0]), int(ks[-1])
    osp = params.get("_output_spatial")
    if osp and len(osp) == 2 and int(osp[0]) > 0 and int(osp[1]) > 0 and int(osp[0]) * int(osp[1]) == hw:
        return n, int(osp[0]), int(osp[1])
    isp = params.get("_input_spatial")
    if isp and len(isp) == 2:
        ho = (int(isp[0]) + pt + pb - dh * (kh - 1) - 1) // sh + 1
        wo = (int(isp[1]) + pl + pr - dw * (kw - 1) - 1) // sw + 1
        if ho > 0 and wo > 0 and ho * wo == hw:
            return n, ho, wo
    h = math.isqrt(hw)
    while h > 0:
        if hw % h == 0:
            w = hw // h
            if (h - 1) * sh - pt - pb + dh * (kh - 1) + 1 > 0 and (w - 1) * sw - pl - pr + dw * (kw - 1) + 1 > 0:
                return n, h, w
        h -= 1
    return None


@register("conv_reshape_f32")
def kernel_conv_reshape(inputs, outputs, params, tuning):
    x = inputs[0]
    if x.ndim == 2:
        geo = conv_output_spatial(x.shape[0], x.shape[1], params)
        if geo is not None:
            n, ho, wo = geo
            o = x.shape[1]
            out = E._planned(_out(outputs), (n, o, ho, wo), x.dtype)
            # out[n, c, h, w] = x[(n*ho + h)*wo + w, c]
            E.strided_copy(x, out, (n, o, ho, wo), [ho * wo * o, 1, wo * o, o])
            outputs[0] = out
            return
    outputs[0] = E.copy_into(x, E._planned(_out(outputs), x.shape, x.dtype))


@register("add_bias_f32")
def kernel_add_bias(inputs, outputs, params, tuning):
    data, bias = inputs[0], inputs[1]
    beta = float(params.get("beta", 1.0))
    axis = int(params.get("bias_axis", -1))
    axis = axis + data.ndim if axis < 0 else axis
    shape = [1] * data.ndim
    shape[axis] = bias.size
    b = bias.reshape(shape)
    outputs[0] = E.run_ew([data, b], [(_lib.EW_MUL_IMM, 1, 1, beta), (_lib.EW_ADD, 0, 2, 0.0)], _out(outputs))


@register("im2col_f32")
def kernel_im2col(inputs, outputs, params, tuning):
    x = inputs[0]
    if x.ndim != 4:
        raise ValueError("im2col requires rank-4 NCHW input")
    kh, kw, sh, sw, dh, dw, pads, ho, wo = E.conv_geometry(x.shape, (0, 0) + tuple(params.get("kernel_shape", [3, 3])),
                                                           {**params, "auto_pad": "NOTSET"})
    n, c, h, w = x.shape
    out = E._planned(_out(outputs), (n * ho * wo, c * kh * kw), x.dtype)
    a = _lib.Im2colArgs()
    a.x, a.out, a.n, a.c, a.h, a.w = x.ptr, out.ptr, n, c, h, w
    a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = kh, kw, sh, sw, pads[0], pads[1], dh, dw, ho, wo
    a.dtype = x.code
    if out.size:
        _lib.launch(a, current_stream())
    outputs[0] = out


@register("winograd_forward_f32")
def kernel_winograd_forward(inputs, outputs, params, tuning):
    """Conv semantics for the 3x3 s1 step; the reference's body cannot compute
    padded convolutions (R:540-566), so this launches the implicit-GEMM conv."""
    outputs[0] = E.conv2d_nchw(inputs[0], inputs[1], None, {**params, **_out(outputs)})


@register("batchnorm_f32")
def kernel_batchnorm(inputs, outputs, params, tuning):
    outputs[0] = E.op_batchnorm(inputs[:5], {"epsilon": params.get("epsilon", 1e-5), **_out(outputs)})


# -- fused ops (R:591-662, delegated to the engine without a temporary) ----------------------------
def _fused(op_type: str):
    def fn(inputs, outputs, params, tuning):
        outputs[0] = E.execute_op(op_type, inputs, {**params, **_out(outputs)})
    return fn


register("fused_matmul_bias_f32")(_fused("FusedMatMulBias"))
register("fused_ew_f32")(_fused("FusedEWChain"))
register("fused_softmax_f32")(_fused("FusedSoftmaxDropout"))
register("fused_residual_norm_f32")(_fused("FusedResidualNorm"))
register("fused_gemm_epilogue_f32")(_fused("FusedGemmEpilogue"))
register("fused_attention_scores_f32")(_fused("FusedAttentionScores"))
register("fused_layer_norm_f32")(_fused("FusedLayerNormalization"))
register("fused_transpose_reshape_f32")(_fused("FusedTransposeReshape"))


@register("fused_residual_relu_f32")
def kernel_fused_residual_relu(inputs, outputs, params, tuning):
    outputs[0] = E.op_fused_residual_relu(inputs[:2], _out(outputs))


# -- metadata / data movement (R:669-759) ---------------------------------------------------------
@register("reshape")
def kernel_reshape(inputs, outputs, params, tuning):
    x = inputs[0]
    if len(inputs) >= 2 and inputs[1] is not None and inputs[1].size > 0:
        shape = E.resolve_reshape_shape(x.shape, E.to_host_ints(inputs[1]), int(params.get("allowzero", 0)))
    else:
        shape = tuple(params.get("_reshape_shape", x.shape))
    out = E._planned(_out(outputs), shape, np.float32)
    outputs[0] = E.cast_into(x.reshape(shape), out)


@register("transpose")
def kernel_transpose(inputs, outputs, params, tuning):
    x = inputs[0]
    perm = params.get("perm")
    perm = list(range(x.ndim - 1, -1, -1)) if perm is None else [int(p) for p in perm]
    outputs[0] = E.transpose(x, perm, _out(outputs))


@register("flatten")
def kernel_flatten(inputs, outputs, params, tuning):
    outputs[0] = E.op_flatten(inputs, {"axis": params.get("axis", 1), **_out(outputs)})


@register("split")
def kernel_split(inputs, outputs, params, tuning):
    parts = E.op_split([inputs[0]], {"axis": params.get("axis", 0), "split": params.get("split", []),
                                     "_num_outputs": int(params.get("_num_outputs", len(outputs))),
                                     "_planned_outputs": list(outputs)})
    for i, p in enumerate(parts):
        if i < len(outputs):
            outputs[i] = p


@register("gather")
def kernel_gather(inputs, outputs, params, tuning):
    """take(x, int64 indices, axis), result as float32 (R:744-752)."""
    outputs[0] = E.gather(inputs[0], inputs[1], int(params.get("axis", 0)), _out(outputs), out_dtype=np.float32)


@register("constant")
def kernel_constant(inputs, outputs, params, tuning):
    pass  # constants are resident via their H2D transfer


# -- rows the reference lacks --------------------------------------------------------------------
@register("maxpool_f32")
def kernel_maxpool(inputs, outputs, params, tuning):
    outputs[0] = E.op_maxpool(inputs[:1], {**params, **_out(outputs)})


@register("quantize_linear")
def kernel_quantize_linear(inputs, outputs, params, tuning):
    outputs[0] = E.op_quantize_linear(inputs, {**params, **_out(outputs)})


@register("qlinear_matmul")
def kernel_qlinear_matmul(inputs, outputs, params, tuning):
    outputs[0] = E.op_qlinear_matmul(inputs, {**params, **_out(outputs)})


@register("dequantize_linear")
def kernel_dequantize_linear(inputs, outputs, params, tuning):
    outputs[0] = E.op_dequantize_linear(inputs, {**params, **_out(outputs)})


@register("argmax")
def kernel_argmax(inputs, outputs, params, tuning):
    outputs[0] = E.op_argmax(inputs[:1], {**params, **_out(outputs)})
