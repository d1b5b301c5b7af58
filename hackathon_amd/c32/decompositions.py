"""Per-op lowering into kernel steps (counterpart of c32/decompositions.py).

Every function returns the ordered KernelSpecRef list the C3.4 planner turns
into kernel steps.  Kernel names, step order, intermediate-tensor names
(`__c3_inter_<node>_<i>__`) and operator_params follow the reference table
(c32/decompositions.py:14-600) exactly, because they are the contract the
registry, the planner and the plan validator key on.  Rows the reference
lacks (MaxPool, BatchNormalization, QuantizeLinear, QLinearMatMul,
DequantizeLinear, ArgMax - the reference's generic fallback names for these
fail closed in its registry) are added with new kernel names.
"""

from __future__ import annotations

from typing import Any, List

from ..c3common.ir.graph import Graph, Node
from .kernel_spec import KernelSpecRef, PrecisionProfile


def _inter_name(node_id: str, idx: int) -> str:
    return f"__c3_inter_{node_id}_{idx}__"


def _kernel_name(base: str, precision: PrecisionProfile) -> str:
    """base + precision suffix with fp32/fp16/fp8 spelled f32/f16/f8."""
    dt = precision.compute_dtype
    return f"{base}_{dt.replace('fp', 'f') if dt.startswith('fp') else dt}"


def _single(node: Node, name: str, params: Any = None) -> List[KernelSpecRef]:
    return [KernelSpecRef(kernel_name=name, inputs=list(node.inputs), outputs=list(node.outputs),
                          operator_params=dict(node.attributes) if params is None else params)]


# -- elementwise ---------------------------------------------------------------
def decompose_Add(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("add", precision), {})


def decompose_Mul(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("mul", precision), {})


def decompose_Div(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("div", precision), {})


def decompose_Relu(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("relu", precision), {})


def decompose_Erf(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("erf", precision), {})


# -- layout / data movement ---------------------------------------------------------
def decompose_Flatten(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "flatten", {"axis": int(node.attributes.get("axis", 1))})


def decompose_Reshape(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "reshape", {"allowzero": int(node.attributes.get("allowzero", 0))})


def decompose_Transpose(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    perm = node.attributes.get("perm")
    return _single(node, "transpose", {"perm": None if perm is None else list(perm)})


def decompose_Split(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    sizes = list(node.attributes.get("split", [])) if "split" in node.attributes else []
    return _single(node, "split", {"axis": int(node.attributes.get("axis", 0)), "split": sizes,
                                   "_num_outputs": len(node.outputs)})


def decompose_Gather(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "gather", {"axis": int(node.attributes.get("axis", 0))})


def decompose_Constant(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return [KernelSpecRef(kernel_name="constant", inputs=[], outputs=list(node.outputs),
                          operator_params=dict(node.attributes))]


# -- MatMul / Gemm --------------------------------------------------------------
def decompose_MatMul(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("matmul", precision), {"lowering_kind": "matmul"})


def decompose_Gemm(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    """alpha*A'B' (+ beta*C as a separate add_bias step when C is present)."""
    attrs = node.attributes
    params = {"alpha": float(attrs.get("alpha", 1.0)), "beta": float(attrs.get("beta", 1.0)),
              "transA": int(attrs.get("transA", 0)), "transB": int(attrs.get("transB", 0)),
              "lowering_kind": "gemm"}
    matmul = _kernel_name("matmul", precision)
    if len(node.inputs) >= 3 and node.inputs[2]:
        tmp = _inter_name(node.id, 0)
        return [
            KernelSpecRef(kernel_name=matmul, inputs=list(node.inputs[:2]), outputs=[tmp],
                          operator_params=dict(params)),
            KernelSpecRef(kernel_name=_kernel_name("add_bias", precision), inputs=[tmp, node.inputs[2]],
                          outputs=list(node.outputs),
                          operator_params={"beta": params["beta"], "bias_axis": -1}),
        ]
    return [KernelSpecRef(kernel_name=matmul, inputs=list(node.inputs[:2]), outputs=list(node.outputs),
                          operator_params=dict(params))]


def decompose_Linear(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    if len(node.inputs) >= 3 and node.inputs[2]:
        return decompose_Gemm(node, graph, precision)
    return decompose_MatMul(node, graph, precision)


# -- Softmax / LayerNorm (unfused) ----------------------------------------------------
def decompose_Softmax(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    nid, x, y = node.id, node.inputs[0], node.outputs[0]
    axis = int(node.attributes.get("axis", -1))
    t = [_inter_name(nid, i) for i in range(4)]
    red = {"axis": axis, "keepdims": True}
    return [
        KernelSpecRef("reduce_max", [x], [t[0]], operator_params=dict(red)),
        KernelSpecRef("sub", [x, t[0]], [t[1]]),
        KernelSpecRef("exp", [t[1]], [t[2]]),
        KernelSpecRef("reduce_sum", [t[2]], [t[3]], operator_params=dict(red)),
        KernelSpecRef("div", [t[2], t[3]], [y]),
    ]


def decompose_LayerNormalization(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    nid, x, y = node.id, node.inputs[0], node.outputs[0]
    weight = node.inputs[1] if len(node.inputs) > 1 else None
    bias = node.inputs[2] if len(node.inputs) > 2 else None
    axis = int(node.attributes.get("axis", -1))
    eps = float(node.attributes.get("epsilon", 1e-5))
    mean = node.outputs[1] if len(node.outputs) > 1 else _inter_name(nid, 0)
    centered, sq, var, var_eps = (_inter_name(nid, i) for i in (1, 2, 3, 4))
    denom, normalized = _inter_name(nid, 5), _inter_name(nid, 6)
    red = {"axis": axis, "axes_from": axis, "keepdims": True}
    refs = [
        KernelSpecRef("reduce_mean", [x], [mean], operator_params=dict(red)),
        KernelSpecRef("sub", [x, mean], [centered]),
        KernelSpecRef("mul", [centered, centered], [sq]),
        KernelSpecRef("reduce_mean", [sq], [var], operator_params=dict(red)),
        KernelSpecRef("add", [var], [var_eps], operator_params={"epsilon": eps}),
        KernelSpecRef("sqrt", [var_eps], [denom]),
    ]
    if len(node.outputs) > 2:
        inv_std = node.outputs[2]
        refs += [KernelSpecRef("reciprocal", [denom], [inv_std]),
                 KernelSpecRef("mul", [centered, inv_std], [normalized])]
    else:
        refs.append(KernelSpecRef("div", [centered, denom], [normalized]))
    if weight:
        refs.append(KernelSpecRef("mul", [normalized, weight], [_inter_name(nid, 7)] if bias else [y]))
    if bias:
        refs.append(KernelSpecRef("add", [_inter_name(nid, 7) if weight else normalized, bias], [y]))
    if not weight and not bias:
        refs[-1].outputs = [y]
    return refs


# -- Conv -----------------------------------------------------------------------
def _conv_kernel_shape(node: Node, graph: Graph) -> List[int]:
    ks = list(node.attributes.get("kernel_shape", []))
    if ks:
        return [int(v) for v in ks]
    if len(node.inputs) > 1:
        w = graph.get_tensor(node.inputs[1])
        if w is not None and len(w.shape) >= 3:
            try:
                return [int(v) for v in w.shape[2:]]
            except (TypeError, ValueError):
                pass
    return []


def _conv_is_winograd_eligible(node: Node, graph: Graph) -> bool:
    ks = _conv_kernel_shape(node, graph)
    return (ks in ([3, 3], [3])
            and list(node.attributes.get("strides", [1, 1])) in ([1], [1, 1])
            and list(node.attributes.get("dilations", [1, 1])) in ([1], [1, 1])
            and int(node.attributes.get("group", 1)) == 1)


def _conv_output_spatial(node: Node, graph: Graph, inp) -> List[int]:
    try:
        if inp is None or len(inp.shape) != 4:
            return []
        h, w = int(inp.shape[-2]), int(inp.shape[-1])
    except (TypeError, ValueError):
        return []
    ks = _conv_kernel_shape(node, graph)
    kh, kw = int(ks[0]), int(ks[-1])
    a = node.attributes
    s, d = list(a.get("strides", [1, 1])), list(a.get("dilations", [1, 1]))
    pt, pl, pb, pr = [int(p) for p in a.get("pads", [0, 0, 0, 0])]
    ho = (h + pt + pb - int(d[0]) * (kh - 1) - 1) // int(s[0]) + 1
    wo = (w + pl + pr - int(d[-1]) * (kw - 1) - 1) // int(s[-1]) + 1
    return [ho, wo] if ho > 0 and wo > 0 else []


def decompose_Conv(node: Node, graph: Graph, precision: PrecisionProfile,
                   use_winograd: bool = True) -> List[KernelSpecRef]:
    """Winograd step for 3x3 s1 convs, else im2col -> contract -> reshape (-> bias)."""
    nid, x, w = node.id, node.inputs[0], node.inputs[1]
    has_bias = len(node.inputs) >= 3 and bool(node.inputs[2])
    a = node.attributes
    conv = {"kernel_shape": _conv_kernel_shape(node, graph), "auto_pad": a.get("auto_pad", "NOTSET"),
            "pads": list(a.get("pads", [0, 0, 0, 0])), "strides": list(a.get("strides", [1, 1])),
            "dilations": list(a.get("dilations", [1, 1])), "group": int(a.get("group", 1))}
    if use_winograd and _conv_is_winograd_eligible(node, graph):
        out = _inter_name(nid, 0) if has_bias else node.outputs[0]
        refs = [KernelSpecRef(_kernel_name("winograd_forward", precision), [x, w],
                              [out] if has_bias else list(node.outputs), operator_params=dict(conv))]
        if has_bias:
            refs.append(KernelSpecRef(_kernel_name("add_bias", precision), [out, node.inputs[2]],
                                      list(node.outputs), operator_params={"bias_axis": 1}))
        return refs
    cols, contract = _inter_name(nid, 0), _inter_name(nid, 1)
    tin = graph.get_tensor(x)
    in_spatial = list(tin.shape[-2:]) if tin is not None and len(tin.shape) == 4 else []
    out_spatial = _conv_output_spatial(node, graph, tin)
    reshape_params = {**conv, "_input_spatial": in_spatial, "_output_spatial": out_spatial}
    refs = [
        KernelSpecRef(_kernel_name("im2col", precision), [x], [cols],
                      operator_params={**conv, "lowering_kind": "conv_im2col"}),
        KernelSpecRef(_kernel_name("matmul", precision), [cols, w], [contract],
                      operator_params={**conv, "lowering_kind": "conv_contract", "_input_spatial": in_spatial}),
    ]
    if has_bias:
        shaped = _inter_name(nid, 2)
        refs += [KernelSpecRef(_kernel_name("conv_reshape", precision), [contract], [shaped],
                               operator_params=dict(reshape_params)),
                 KernelSpecRef(_kernel_name("add_bias", precision), [shaped, node.inputs[2]],
                               list(node.outputs), operator_params={"bias_axis": 1})]
    else:
        refs.append(KernelSpecRef(_kernel_name("conv_reshape", precision), [contract], list(node.outputs),
                                  operator_params=dict(reshape_params)))
    return refs


def decompose_GlobalAveragePool(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, _kernel_name("reduce_mean", precision), {"axes": [-2, -1], "keepdims": True})


# -- C3.3 fused nodes ------------------------------------------------------------
def decompose_FusedMatMulBias(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_matmul_bias_f32")


def decompose_FusedConv2dBatchNorm(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    """Folded: plain Conv lowering.  Unfolded: Conv lowering + batchnorm step."""
    if node.attributes.get("bn_folded"):
        return decompose_Conv(node, graph, precision, use_winograd=True)
    offset = int(node.attributes.get("bn_parameter_offset", len(node.inputs)))
    conv_out = _inter_name(node.id, 0)
    conv = Node(id=f"{node.id}_conv", name=node.name, op_type="Conv", inputs=list(node.inputs[:offset]),
                outputs=[conv_out], attributes=dict(node.attributes), domain=node.domain)
    refs = decompose_Conv(conv, graph, precision, use_winograd=True)
    refs.append(KernelSpecRef("batchnorm_f32", [conv_out] + list(node.inputs[offset:offset + 4]),
                              list(node.outputs),
                              operator_params={"epsilon": node.attributes.get("bn_epsilon", 1e-5)}))
    return refs


def decompose_FusedEWChain(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_ew_f32")


def decompose_FusedSoftmaxDropout(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_softmax_f32")


def decompose_FusedResidualNorm(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_residual_norm_f32")


def decompose_FusedGemmEpilogue(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_gemm_epilogue_f32")


def _conv_epilogue(node: Node, graph: Graph, precision: PrecisionProfile, residual: bool) -> List[KernelSpecRef]:
    end = len(node.inputs)
    if residual:
        end = int(node.attributes.get("_residual_input_index", len(node.inputs)))
        if not 0 <= end < len(node.inputs):
            raise ValueError("Fused Conv residual input index is invalid")
    conv_out = _inter_name(node.id, 2)
    conv = Node(id=f"{node.id}_blas_conv", name=node.name, op_type="Conv", inputs=list(node.inputs[:end]),
                outputs=[conv_out], attributes=dict(node.attributes), domain=node.domain)
    refs = decompose_Conv(conv, graph, precision, use_winograd=False)
    if residual:
        refs.append(KernelSpecRef("fused_residual_relu_f32", [conv_out, node.inputs[end]], list(node.outputs),
                                  operator_params={"lowering_kind": "blas_conv_residual_relu_epilogue"}))
    else:
        refs.append(KernelSpecRef("relu_f32", [conv_out], list(node.outputs),
                                  operator_params={"lowering_kind": "blas_conv_relu_epilogue"}))
    return refs


def decompose_FusedConvActivation(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _conv_epilogue(node, graph, precision, residual=False)


def decompose_FusedConvResidualActivation(node: Node, graph: Graph,
                                          precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _conv_epilogue(node, graph, precision, residual=True)


def decompose_FusedAttentionScores(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_attention_scores_f32")


def decompose_FusedLayerNormalization(node: Node, graph: Graph,
                                      precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_layer_norm_f32")


def decompose_FusedTransposeReshape(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "fused_transpose_reshape_f32")


# -- rows the reference lacks ----------------------------------------------------------
def decompose_MaxPool(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    """ONNX MaxPool (padding acts as -inf): one `maxpool_f32` step."""
    a = node.attributes
    ks = [int(v) for v in a.get("kernel_shape", [])]
    params = {"kernel_shape": ks, "pads": list(a.get("pads", [0] * (2 * len(ks)))),
              "strides": list(a.get("strides", [1] * len(ks))),
              "dilations": list(a.get("dilations", [1] * len(ks))),
              "ceil_mode": int(a.get("ceil_mode", 0)), "auto_pad": a.get("auto_pad", "NOTSET")}
    return _single(node, "maxpool_f32", params)


def decompose_BatchNormalization(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "batchnorm_f32", {"epsilon": float(node.attributes.get("epsilon", 1e-5))})


def decompose_QuantizeLinear(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "quantize_linear", {"axis": int(node.attributes.get("axis", 1))})


def decompose_DequantizeLinear(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "dequantize_linear", {"axis": int(node.attributes.get("axis", 1))})


def decompose_QLinearMatMul(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    return _single(node, "qlinear_matmul", {})


def decompose_ArgMax(node: Node, graph: Graph, precision: PrecisionProfile) -> List[KernelSpecRef]:
    a = node.attributes
    return _single(node, "argmax", {"axis": int(a.get("axis", 0)), "keepdims": int(a.get("keepdims", 1)),
                                    "select_last_index": int(a.get("select_last_index", 0))})


DECOMPOSE_DISPATCH = {
    "Add": decompose_Add,
    "Constant": decompose_Constant,
    "Conv": decompose_Conv,
    "Conv2d": decompose_Conv,
    "Div": decompose_Div,
    "Erf": decompose_Erf,
    "Flatten": decompose_Flatten,
    "FusedConv2dBatchNorm": decompose_FusedConv2dBatchNorm,
    "FusedConvActivation": decompose_FusedConvActivation,
    "FusedConvResidualActivation": decompose_FusedConvResidualActivation,
    "FusedAttentionScores": decompose_FusedAttentionScores,
    "FusedEWChain": decompose_FusedEWChain,
    "FusedGemmEpilogue": decompose_FusedGemmEpilogue,
    "FusedLayerNormalization": decompose_FusedLayerNormalization,
    "FusedTransposeReshape": decompose_FusedTransposeReshape,
    "FusedMatMulBias": decompose_FusedMatMulBias,
    "FusedResidualNorm": decompose_FusedResidualNorm,
    "FusedSoftmaxDropout": decompose_FusedSoftmaxDropout,
    "Gather": decompose_Gather,
    "Gemm": decompose_Gemm,
    "GlobalAveragePool": decompose_GlobalAveragePool,
    "LayerNormalization": decompose_LayerNormalization,
    "LayerNorm": decompose_LayerNormalization,
    "Linear": decompose_Linear,
    "MatMul": decompose_MatMul,
    "Mul": decompose_Mul,
    "Relu": decompose_Relu,
    "Reshape": decompose_Reshape,
    "Softmax": decompose_Softmax,
    "Split": decompose_Split,
    "Transpose": decompose_Transpose,
    # Added rows (no counterpart in the reference table).
    "MaxPool": decompose_MaxPool,
    "BatchNormalization": decompose_BatchNormalization,
    "QuantizeLinear": decompose_QuantizeLinear,
    "DequantizeLinear": decompose_DequantizeLinear,
    "QLinearMatMul": decompose_QLinearMatMul,
    "ArgMax": decompose_ArgMax,
}
