"""The five BASELINE workloads, built in-script as C3 graphs with seeded weights.

The reference imports ONNX files (c31/import_onnx.py:59-240); the `onnx`
package is not available on these machines, so each model is built directly
as the graph an ONNX exporter would produce (same op types, attributes,
initializer roles and tensor metadata), with weights drawn from
`numpy.random.default_rng(seed)` in graph order: inputs first, then
parameters layer by layer.  `hackathon_amd.onnx_io` writes/reads the same
graphs as real .onnx files.

Configs (BASELINE.json:7-11):
  1 mlp            784-512-256-10 Gemm/ReLU, fp32, B=256
  2 resnet18_cifar ResNet-18 (3x3 stem, no max-pool), explicit BN, fp32, B=256, 32x32
  3 resnet18_224   ResNet-18 (7x7/2 stem + max-pool), bf16 policy, B=256, 224x224
  4 decoder_fp16   6 layers, d=512, 8 heads, FFN 2048 GELU, pre-LN, vocab 8192, S=256, B=64
  5 decoder_w8a8   12 layers, d=768, 12 heads, FFN 3072, vocab 32000, S=1024, B=16, W8A8 Linear
Extra workload (not a BASELINE config):
    decoder_fp8    config 4's model under the "fp8" policy (E4M3 GEMMs for every
                   aligned constant-weight Linear, fp16 elsewhere)
    decoder_fp4    config 4's model under the "fp4" policy (W4A16 GEMMs -- MXFP4
                   weights, fp16 activations -- for the large aligned
                   constant-weight Linears, fp16 elsewhere)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .c3common.ir.graph import Graph, Node, ONNSType

_NP_TO_ONNS = {
    np.dtype(np.float32): ONNSType.FLOAT, np.dtype(np.float16): ONNSType.FLOAT16,
    np.dtype(np.int64): ONNSType.INT64, np.dtype(np.int32): ONNSType.INT32,
    np.dtype(np.int8): ONNSType.INT8, np.dtype(np.uint8): ONNSType.UINT8,
    np.dtype(np.bool_): ONNSType.BOOL, np.dtype(np.float64): ONNSType.DOUBLE,
}


@dataclass
class Model:
    """A graph plus its initializer payloads and a seeded input batch."""

    name: str
    graph: Graph
    weights: Dict[str, np.ndarray]
    inputs: Dict[str, np.ndarray]
    precision: str = "fp32"          # executable precision policy name
    unit: str = "samples"            # "samples" or "tokens"
    tokens_per_sample: int = 1
    meta: Dict[str, Any] = field(default_factory=dict)


class GraphBuilder:
    """Append-only construction of a C3 graph with ONNX-style naming."""

    def __init__(self, name: str) -> None:
        self.g = Graph()
        self.g.name = name
        self.g.opsets = {"ai.onnx": 17}
        self.weights: Dict[str, np.ndarray] = {}
        self._count: Dict[str, int] = {}

    def fresh(self, prefix: str) -> str:
        n = self._count.get(prefix, 0)
        self._count[prefix] = n + 1
        return f"{prefix}_{n}"

    def input(self, name: str, dtype, shape: Sequence[Any]) -> str:
        t = self.g.register_tensor(name, _NP_TO_ONNS[np.dtype(dtype)], list(shape))
        self.g.inputs.append(t)
        self.g.tensor_producer[name] = "INPUT"
        return name

    def init(self, name: str, value: np.ndarray) -> str:
        value = np.ascontiguousarray(value)
        t = self.g.register_tensor(name, _NP_TO_ONNS[value.dtype], list(value.shape), is_initializer=True)
        self.g.initializers[name] = t
        self.g.tensor_producer[name] = "INITIALIZER"
        self.weights[name] = value
        return name

    def node(self, op: str, inputs: List[str], n_out: int = 1, shape: Optional[Sequence[Any]] = None,
             dtype=np.float32, shapes: Optional[List[Sequence[Any]]] = None, name: Optional[str] = None,
             **attrs: Any) -> Any:
        nid = name or self.fresh(op.lower())
        outs = [f"{nid}_out{i}" if n_out > 1 else f"{nid}_out" for i in range(n_out)]
        node = Node(id=nid, name=nid, op_type=op, inputs=list(inputs), outputs=outs, attributes=dict(attrs))
        self.g.add_node(node)
        for i, o in enumerate(outs):
            shp = shapes[i] if shapes is not None else shape
            self.g.register_tensor(o, _NP_TO_ONNS[np.dtype(dtype)], list(shp) if shp is not None else [])
            self.g.set_producer(o, nid)
        return outs if n_out > 1 else outs[0]

    def output(self, tensor: str, name: str = "logits") -> str:
        """Rename `tensor` to the public output name and mark it a graph output."""
        if tensor != name:
            producer = self.g.nodes[self.g.tensor_producer[tensor]]
            t = self.g.tensors.pop(tensor)
            t.name = name
            self.g.tensors[name] = t
            producer.outputs = [name if o == tensor else o for o in producer.outputs]
            self.g.tensor_producer[name] = self.g.tensor_producer.pop(tensor)
            for nid in self.g.tensor_consumers.pop(tensor, []):
                self.g.nodes[nid].inputs = [name if i == tensor else i for i in self.g.nodes[nid].inputs]
                self.g.add_consumer(name, nid)
        self.g.outputs.append(self.g.tensors[name])
        return name

    def finish(self) -> Graph:
        self.g.validate()
        return self.g


# -- 1: MLP ------------------------------------------------------------------------
def build_mlp(batch: int = 256, dims: Sequence[int] = (784, 512, 256, 10), seed: int = 0) -> Model:
    rng = np.random.default_rng(seed)
    b = GraphBuilder("mlp")
    x = rng.random((batch, dims[0]), dtype=np.float32)
    h = b.input("input", np.float32, ["N", dims[0]])
    for i, (fan_in, fan_out) in enumerate(zip(dims[:-1], dims[1:])):
        w = (rng.standard_normal((fan_out, fan_in), dtype=np.float32) * np.float32(math.sqrt(2.0 / fan_in)))
        wn = b.init(f"fc{i + 1}.weight", w.astype(np.float32))
        bn = b.init(f"fc{i + 1}.bias", np.zeros(fan_out, np.float32))
        h = b.node("Gemm", [h, wn, bn], shape=["N", fan_out], name=f"fc{i + 1}", transB=1, alpha=1.0, beta=1.0)
        if i < len(dims) - 2:
            h = b.node("Relu", [h], shape=["N", fan_out], name=f"relu{i + 1}")
    b.output(h)
    return Model("mlp", b.finish(), b.weights, {"input": x}, precision="fp32")


# -- 2/3: ResNet-18 --------------------------------------------------------------------
def _conv_bn(b: GraphBuilder, rng, x: str, cin: int, cout: int, k: int, stride: int, pad: int,
             hw: Tuple[int, int], prefix: str) -> Tuple[str, Tuple[int, int]]:
    h, w = hw
    ho, wo = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    weight = rng.standard_normal((cout, cin, k, k), dtype=np.float32) * np.float32(math.sqrt(2.0 / (cin * k * k)))
    wn = b.init(f"{prefix}.conv.weight", weight.astype(np.float32))
    y = b.node("Conv", [x, wn], shape=["N", cout, ho, wo], name=f"{prefix}.conv", kernel_shape=[k, k],
               strides=[stride, stride], pads=[pad, pad, pad, pad], dilations=[1, 1], group=1)
    gamma = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    beta = (rng.standard_normal(cout) * 0.1).astype(np.float32)
    mean = (rng.standard_normal(cout) * 0.1).astype(np.float32)
    var = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    names = [b.init(f"{prefix}.bn.{n}", v) for n, v in
             (("weight", gamma), ("bias", beta), ("running_mean", mean), ("running_var", var))]
    y = b.node("BatchNormalization", [y] + names, shape=["N", cout, ho, wo], name=f"{prefix}.bn",
               epsilon=1e-5, momentum=0.9)
    return y, (ho, wo)


def build_resnet18(batch: int = 256, image: int = 32, stem: str = "cifar", classes: int = 10,
                   widths: Sequence[int] = (64, 128, 256, 512), blocks: Sequence[int] = (2, 2, 2, 2),
                   precision: str = "fp32", seed: int = 0, name: Optional[str] = None) -> Model:
    rng = np.random.default_rng(seed)
    b = GraphBuilder(name or f"resnet18_{stem}")
    x = rng.standard_normal((batch, 3, image, image), dtype=np.float32)
    h = b.input("input", np.float32, ["N", 3, image, image])
    hw = (image, image)
    if stem == "cifar":
        h, hw = _conv_bn(b, rng, h, 3, widths[0], 3, 1, 1, hw, "stem")
        h = b.node("Relu", [h], shape=["N", widths[0], *hw], name="stem.relu")
    else:
        h, hw = _conv_bn(b, rng, h, 3, widths[0], 7, 2, 3, hw, "stem")
        h = b.node("Relu", [h], shape=["N", widths[0], *hw], name="stem.relu")
        ho = (hw[0] + 2 - 3) // 2 + 1
        h = b.node("MaxPool", [h], shape=["N", widths[0], ho, ho], name="stem.pool", kernel_shape=[3, 3],
                   strides=[2, 2], pads=[1, 1, 1, 1])
        hw = (ho, ho)
    cin = widths[0]
    for stage, (cout, nblk) in enumerate(zip(widths, blocks)):
        for blk in range(nblk):
            stride = 2 if (stage > 0 and blk == 0) else 1
            p = f"layer{stage + 1}.{blk}"
            y, hw2 = _conv_bn(b, rng, h, cin, cout, 3, stride, 1, hw, f"{p}.a")
            y = b.node("Relu", [y], shape=["N", cout, *hw2], name=f"{p}.a.relu")
            y, hw2 = _conv_bn(b, rng, y, cout, cout, 3, 1, 1, hw2, f"{p}.b")
            if stride != 1 or cin != cout:
                sc, _ = _conv_bn(b, rng, h, cin, cout, 1, stride, 0, hw, f"{p}.down")
            else:
                sc = h
            y = b.node("Add", [y, sc], shape=["N", cout, *hw2], name=f"{p}.add")
            h = b.node("Relu", [y], shape=["N", cout, *hw2], name=f"{p}.relu")
            cin, hw = cout, hw2
    h = b.node("GlobalAveragePool", [h], shape=["N", cin, 1, 1], name="gap")
    h = b.node("Flatten", [h], shape=["N", cin], name="flatten", axis=1)
    w = rng.standard_normal((classes, cin), dtype=np.float32) * np.float32(math.sqrt(2.0 / cin))
    wn = b.init("fc.weight", w.astype(np.float32))
    bn = b.init("fc.bias", np.zeros(classes, np.float32))
    h = b.node("Gemm", [h, wn, bn], shape=["N", classes], name="fc", transB=1, alpha=1.0, beta=1.0)
    b.output(h)
    return Model(b.g.name, b.finish(), b.weights, {"input": x}, precision=precision)


def build_resnet18_cifar(batch: int = 256, **kw: Any) -> Model:
    return build_resnet18(batch=batch, image=kw.pop("image", 32), stem="cifar", classes=kw.pop("classes", 10),
                          precision="fp32", name="resnet18_cifar", **kw)


def build_resnet18_224(batch: int = 256, **kw: Any) -> Model:
    return build_resnet18(batch=batch, image=kw.pop("image", 224), stem="imagenet",
                          classes=kw.pop("classes", 1000), precision=kw.pop("precision", "bf16"),
                          name="resnet18_224", **kw)


# -- 4/5: decoder-only transformers ----------------------------------------------------------
def _causal_mask(seq: int) -> np.ndarray:
    m = np.zeros((1, 1, seq, seq), np.float32)
    m[0, 0][np.triu_indices(seq, 1)] = -np.inf
    return m


def build_decoder(batch: int = 64, seq: int = 256, d_model: int = 512, heads: int = 8, ffn: int = 2048,
                  layers: int = 6, vocab: int = 8192, precision: str = "fp16", quantized: bool = False,
                  seed: int = 0, name: Optional[str] = None,
                  act_scales: Optional[Dict[str, float]] = None, argmax: bool = True) -> Model:
    """Pre-LN decoder; `quantized` routes every Linear through QDQ int8.

    Outputs: "logits" [N, seq, vocab] and, with `argmax`, "argmax" [N, seq]
    (int64, first index of the maximum, ONNX ArgMax axis=-1 keepdims=0)."""
    rng = np.random.default_rng(seed)
    name = name or ("decoder_w8a8" if quantized else "decoder_fp16")
    b = GraphBuilder(name)
    dh = d_model // heads
    ids = rng.integers(0, vocab, size=(batch, seq), dtype=np.int64)
    x_in = b.input("input_ids", np.int64, ["N", seq])

    def normal(shape, std=0.02):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    def const(n: str, v) -> str:
        return b.init(n, np.asarray(v))

    tok = b.init("embed.tok", normal((vocab, d_model)))
    pos = b.init("embed.pos", normal((seq, d_model)))
    h = b.node("Gather", [tok, x_in], shape=["N", seq, d_model], name="embed.gather", axis=0)
    x = b.node("Add", [h, pos], shape=["N", seq, d_model], name="embed.add")
    mask = const("attn.mask", _causal_mask(seq))
    divisor = const("attn.scale", np.array([math.sqrt(dh)], np.float32))
    sqrt2 = const("gelu.sqrt2", np.array([math.sqrt(2.0)], np.float32))
    one = const("gelu.one", np.array([1.0], np.float32))
    half = const("gelu.half", np.array([0.5], np.float32))
    shape_heads = const("shape.heads", np.array([0, 0, heads, dh], np.int64))
    shape_model = const("shape.model", np.array([0, 0, d_model], np.int64))
    quant: List[Tuple[str, str]] = []  # (activation scale name, output scale name) to calibrate

    def ln(inp: str, prefix: str) -> str:
        g = b.init(f"{prefix}.weight", np.ones(d_model, np.float32))
        be = b.init(f"{prefix}.bias", np.zeros(d_model, np.float32))
        return b.node("LayerNormalization", [inp, g, be], shape=["N", seq, d_model], name=prefix, axis=-1,
                      epsilon=1e-5)

    def linear(inp: str, fin: int, fout: int, prefix: str) -> str:
        w = normal((fin, fout))
        bias = b.init(f"{prefix}.bias", np.zeros(fout, np.float32))
        if not quantized:
            wn = b.init(f"{prefix}.weight", w)
            y = b.node("MatMul", [inp, wn], shape=["N", seq, fout], name=f"{prefix}.matmul")
            return b.node("Add", [y, bias], shape=["N", seq, fout], name=f"{prefix}.add")
        sw = (np.max(np.abs(w), axis=0) / 127.0).astype(np.float32)
        wq = np.clip(np.rint(w / sw), -127, 127).astype(np.int8)
        wn = b.init(f"{prefix}.weight_q", wq)
        swn = b.init(f"{prefix}.weight_scale", sw)
        zw = b.init(f"{prefix}.weight_zero", np.zeros(fout, np.int8))
        sa = b.init(f"{prefix}.act_scale", np.array(1.0, np.float32))
        za = b.init(f"{prefix}.act_zero", np.array(0, np.int8))
        sy = b.init(f"{prefix}.out_scale", np.array(1.0, np.float32))
        zy = b.init(f"{prefix}.out_zero", np.array(0, np.int8))
        aq = b.node("QuantizeLinear", [inp, sa, za], shape=["N", seq, fin], dtype=np.int8,
                    name=f"{prefix}.quant")
        yq = b.node("QLinearMatMul", [aq, sa, za, wn, swn, zw, sy, zy], shape=["N", seq, fout], dtype=np.int8,
                    name=f"{prefix}.qmatmul")
        y = b.node("DequantizeLinear", [yq, sy, zy], shape=["N", seq, fout], name=f"{prefix}.dequant")
        quant.append((sa, sy))
        return b.node("Add", [y, bias], shape=["N", seq, fout], name=f"{prefix}.add")

    for li in range(layers):
        p = f"layer{li}"
        hn = ln(x, f"{p}.ln1")
        qkv = linear(hn, d_model, 3 * d_model, f"{p}.qkv")
        q, k, v = b.node("Split", [qkv], n_out=3, shapes=[["N", seq, d_model]] * 3, name=f"{p}.split", axis=-1)
        hs = ["N", seq, heads, dh]
        q = b.node("Reshape", [q, shape_heads], shape=hs, name=f"{p}.q.reshape")
        q = b.node("Transpose", [q], shape=["N", heads, seq, dh], name=f"{p}.q.transpose", perm=[0, 2, 1, 3])
        k = b.node("Reshape", [k, shape_heads], shape=hs, name=f"{p}.k.reshape")
        kt = b.node("Transpose", [k], shape=["N", heads, dh, seq], name=f"{p}.k.transpose", perm=[0, 2, 3, 1])
        v = b.node("Reshape", [v, shape_heads], shape=hs, name=f"{p}.v.reshape")
        v = b.node("Transpose", [v], shape=["N", heads, seq, dh], name=f"{p}.v.transpose", perm=[0, 2, 1, 3])
        s = b.node("MatMul", [q, kt], shape=["N", heads, seq, seq], name=f"{p}.scores")
        s = b.node("Div", [s, divisor], shape=["N", heads, seq, seq], name=f"{p}.scale")
        s = b.node("Add", [s, mask], shape=["N", heads, seq, seq], name=f"{p}.mask")
        pr = b.node("Softmax", [s], shape=["N", heads, seq, seq], name=f"{p}.softmax", axis=-1)
        ctx = b.node("MatMul", [pr, v], shape=["N", heads, seq, dh], name=f"{p}.context")
        ctx = b.node("Transpose", [ctx], shape=["N", seq, heads, dh], name=f"{p}.ctx.transpose", perm=[0, 2, 1, 3])
        ctx = b.node("Reshape", [ctx, shape_model], shape=["N", seq, d_model], name=f"{p}.ctx.reshape")
        o = linear(ctx, d_model, d_model, f"{p}.out")
        x = b.node("Add", [x, o], shape=["N", seq, d_model], name=f"{p}.residual1")
        hn = ln(x, f"{p}.ln2")
        f = linear(hn, d_model, ffn, f"{p}.ffn1")
        g = b.node("Div", [f, sqrt2], shape=["N", seq, ffn], name=f"{p}.gelu.div")
        g = b.node("Erf", [g], shape=["N", seq, ffn], name=f"{p}.gelu.erf")
        g = b.node("Add", [g, one], shape=["N", seq, ffn], name=f"{p}.gelu.add")
        g = b.node("Mul", [f, g], shape=["N", seq, ffn], name=f"{p}.gelu.mul")
        g = b.node("Mul", [g, half], shape=["N", seq, ffn], name=f"{p}.gelu.half")
        f = linear(g, ffn, d_model, f"{p}.ffn2")
        x = b.node("Add", [x, f], shape=["N", seq, d_model], name=f"{p}.residual2")
    hn = ln(x, "final.ln")
    logits = b.output(linear(hn, d_model, vocab, "lm_head"))
    if argmax:  # the predicted token per position ("output logits + argmax")
        pred = b.node("ArgMax", [logits], shape=["N", seq], dtype=np.int64, name="predict", axis=-1, keepdims=0)
        b.output(pred, "argmax")
    signature = f"b{batch}_s{seq}_d{d_model}_h{heads}_f{ffn}_l{layers}_v{vocab}_seed{seed}"
    model = Model(name, b.finish(), b.weights, {"input_ids": ids},
                  precision="w8a8" if quantized else precision, unit="tokens", tokens_per_sample=seq,
                  meta={"heads": heads, "d_model": d_model, "seq": seq, "layers": layers, "vocab": vocab,
                        "quant_scales": [n for pair in quant for n in pair], "signature": signature})
    if quantized:
        if act_scales is not None:
            apply_activation_scales(model, act_scales)
        else:
            load_activation_scales(model)
    return model


CALIBRATION_DIR = __import__("pathlib").Path(__file__).resolve().parent / "calibration"


def calibration_path(name: str):
    return CALIBRATION_DIR / f"{name}.json"


def apply_activation_scales(model: Model, scales: Dict[str, float]) -> None:
    """Install per-tensor activation/output scales (name -> scale) into the weights."""
    missing = [n for n in model.meta["quant_scales"] if n not in scales]
    if missing:
        raise ValueError(f"calibration lacks scales for {missing[:4]}...")
    for n in model.meta["quant_scales"]:
        model.weights[n] = np.array(scales[n], np.float32)


def load_activation_scales(model: Model) -> None:
    """Load committed calibration scales for a full-size W8A8 model.

    The scales come from a float calibration forward of the first sample
    (max|x|/127 per QuantizeLinear input and QLinearMatMul output with QDQ
    bypassed), produced once by tests/golden/make_w8a8_calibration.py and
    committed as data; building the model never runs that forward.
    """
    import json

    path = calibration_path(model.name)
    if not path.exists():
        raise FileNotFoundError(f"no committed calibration for {model.name}: {path}")
    data = json.loads(path.read_text())
    if data.get("signature") != model.meta["signature"]:
        raise ValueError(f"calibration {path} was made for {data.get('signature')}, not {model.meta['signature']}")
    apply_activation_scales(model, data["scales"])


CONFIGS: Dict[str, Callable[..., Model]] = {
    "mlp": build_mlp,
    "resnet18_cifar": build_resnet18_cifar,
    "resnet18_224": build_resnet18_224,
    "decoder_fp16": lambda **kw: build_decoder(**{"precision": "fp16", **kw}),
    "decoder_fp8": lambda **kw: build_decoder(**{"precision": "fp8", "name": "decoder_fp8", **kw}),
    "decoder_fp4": lambda **kw: build_decoder(**{"precision": "fp4", "name": "decoder_fp4", **kw}),
    "decoder_w8a8": lambda **kw: build_decoder(**{"batch": 16, "seq": 1024, "d_model": 768, "heads": 12,
                                                  "ffn": 3072, "layers": 12, "vocab": 32000,
                                                  "quantized": True, **kw}),
}

CONFIG_ORDER = ["mlp", "resnet18_cifar", "resnet18_224", "decoder_fp16", "decoder_w8a8"]


def build(config: str, **kw: Any) -> Model:
    return CONFIGS[config](**kw)
