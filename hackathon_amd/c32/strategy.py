"""Precision selection, decomposition and tuning (counterpart of c32/strategy.py).

`Strategy` keeps the reference's public methods and rules
(c32/strategy.py:51-354): FULL_FP32 forces fp32 everywhere; sensitive ops
stay fp32; decompositions are validated for connectivity; tuning formulas are
the reference's.  The reference planner can only emit FULL_FP32 plans
(c34/scheduler.py:70), so this build adds an explicit `PrecisionPolicy` that
the planner passes through to `KernelStep.precision_profile`:

  * "fp32"  - the reference behaviour;
  * "bf16" / "fp16" - contractions (Conv, Gemm, MatMul and their fused forms)
    compute in the 16-bit type with fp32 accumulation; every floating
    activation is stored in the 16-bit type; sensitive ops (LayerNorm,
    Softmax, attention) compute in fp32 from 16-bit storage; graph outputs
    are fp32;
  * "w8a8" - QLinearMatMul computes int8 x int8 -> int32; float activations
    are stored in bf16 as in "bf16";
  * "fp8"  - the executable form of the reference's mixed-precision choice
    (c32/strategy.py:124-160) on a profile without fp4: a constant-weight
    GEMM that the reference's rule gives fp8 (or fp4, which then falls back
    to fp8, c32/strategy.py:113-122) computes OCP E4M3 x E4M3 with fp32
    accumulation (row-wise dynamic activation scales, per-output-channel
    weight scales); every other contraction, and every activation in
    storage, is fp16.  The reference also picks fp8 for aligned 1x1 convs;
    no fp8 conv kernel exists here, so those run fp16.
  * "fp4"  - the same rule on this profile, which declares fp4: the large
    aligned constant-weight GEMMs it gives fp4 (c32/strategy.py:150-154) run
    W4A16 -- MXFP4 weights (E2M1, one E8M0 exponent per 32 k) widened to
    fp16 in registers, fp16 activations, fp32 accumulation
    (c32/strategy.py:101-108); those it gives fp8 run E4M3 as under "fp8";
    the rest, and every activation in storage, fp16.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Any, Dict, List, Optional, Set

from ..c3common.ir.graph import Graph, Node
from .decompositions import DECOMPOSE_DISPATCH
from .hardware import HardwareCapability, get_hardware
from .kernel_spec import KernelSpecRef, KernelTuningParams, PrecisionProfile, ProblemSize


class ExecutionMode(str, Enum):
    FULL_FP32 = "FULL_FP32"
    MIXED_PRECISION = "MIXED_PRECISION"


SENSITIVE_OPS: Set[str] = {
    "Softmax", "LogSoftmax", "LayerNorm", "LayerNormalization", "BatchNorm", "BatchNormalization",
    "ReduceMax", "ReduceSum", "ReduceMean", "FusedAttentionScores", "FusedLayerNormalization",
    "FusedResidualNorm", "FusedSoftmaxDropout",
}

TUNABLE_OPS: Set[str] = {"MatMul", "Linear", "Gemm", "Conv", "Conv2d"}

# Contractions under a 16-bit / int8 policy (the fused forms included, which
# the reference's TUNABLE_OPS misses, c32/strategy.py:33).
CONTRACTION_OPS: Set[str] = TUNABLE_OPS | {
    "FusedConv2dBatchNorm", "FusedConvActivation", "FusedConvResidualActivation",
    "FusedMatMulBias", "FusedGemmEpilogue",
}

SAFE_FALLBACKS: Dict[str, List[str]] = {
    "fp4": ["fp4", "fp8", "fp16", "bf16", "fp32"],
    "fp8": ["fp8", "fp16", "bf16", "fp32"],
    "fp16": ["fp16", "bf16", "fp32"],
    "bf16": ["bf16", "fp16", "fp32"],
    "fp32": ["fp32"],
}

METADATA_KERNELS: Set[str] = {"constant", "flatten", "reshape", "transpose", "split", "gather"}


POLICY_NAMES = ("fp32", "bf16", "fp16", "w8a8", "fp8", "fp4")


@dataclass(frozen=True)
class PrecisionPolicy:
    """Executable precision policy (name in {"fp32", "bf16", "fp16", "w8a8", "fp8", "fp4"})."""

    name: str = "fp32"

    def __post_init__(self) -> None:
        if self.name not in POLICY_NAMES:
            raise ValueError(f"unknown precision policy {self.name!r}")

    @property
    def activation_dtype(self) -> str:
        return {"fp32": "fp32", "bf16": "bf16", "fp16": "fp16", "w8a8": "bf16", "fp8": "fp16",
                "fp4": "fp16"}[self.name]

    @property
    def contraction_dtype(self) -> str:
        """Contraction type of nodes the policy does not single out (fp8, fp4: the fp16 fallback)."""
        return {"fp32": "fp32", "bf16": "bf16", "fp16": "fp16", "w8a8": "bf16", "fp8": "fp16",
                "fp4": "fp16"}[self.name]


FP32_POLICY = PrecisionPolicy("fp32")


class Strategy:
    def __init__(self, hardware: Optional[HardwareCapability] = None,
                 mode: ExecutionMode = ExecutionMode.FULL_FP32,
                 policy: Optional[PrecisionPolicy] = None) -> None:
        self._hardware_arg = hardware
        self.hardware = hardware or get_hardware()
        self.mode = ExecutionMode(mode)
        self.policy = policy or FP32_POLICY

    def refresh_hardware(self) -> None:
        if self._hardware_arg is None:
            self.hardware = get_hardware()

    # -- precision ----------------------------------------------------------------
    def select_precision(self, node: Node, graph: Graph) -> PrecisionProfile:
        if self.policy.name != "fp32":
            return self._policy_precision(node, graph)
        if self.mode == ExecutionMode.FULL_FP32 or node.op_type in SENSITIVE_OPS:
            return PrecisionProfile()
        if node.op_type in TUNABLE_OPS:
            chosen = self._supported_fallback(self._preferred_tunable_precision(node, graph))
            act = "fp16" if chosen == "fp4" else chosen
            return PrecisionProfile(compute_dtype=chosen, accumulator_dtype="fp32", input_dtype=act,
                                    weight_dtype=chosen, output_dtype="fp32")
        return PrecisionProfile()

    def _policy_precision(self, node: Node, graph: Graph) -> PrecisionProfile:
        act = self.policy.activation_dtype
        graph_outputs = {t.name for t in graph.outputs}
        out = "fp32" if any(o in graph_outputs for o in node.outputs) else act
        if node.op_type == "QLinearMatMul":
            return PrecisionProfile(compute_dtype="int8", accumulator_dtype="int8", input_dtype="int8",
                                    weight_dtype="int8", output_dtype="int8")
        if node.op_type == "QuantizeLinear":
            return PrecisionProfile(compute_dtype="fp32", input_dtype=act, output_dtype="int8")
        if node.op_type == "DequantizeLinear":
            return PrecisionProfile(compute_dtype="fp32", input_dtype="int8", output_dtype=out)
        if node.op_type in CONTRACTION_OPS:
            low = self.executable_low_precision(node, graph)
            if low == "fp4":
                return PrecisionProfile(compute_dtype="fp4", accumulator_dtype="fp32", input_dtype="fp16",
                                        weight_dtype="fp4", output_dtype=out)
            if low == "fp8":
                return PrecisionProfile(compute_dtype="fp8", accumulator_dtype="fp32", input_dtype="fp8",
                                        weight_dtype="fp8", output_dtype=out)
            c = self.policy.contraction_dtype
            return PrecisionProfile(compute_dtype=c, accumulator_dtype="fp32", input_dtype=act,
                                    weight_dtype=c, output_dtype=out)
        return PrecisionProfile(compute_dtype="fp32", accumulator_dtype="fp32", input_dtype=act,
                                output_dtype=out)

    def _supported_fallback(self, preferred: str, allow_fp4: bool = True) -> str:
        supported = set(self.hardware.supported_precisions())
        if not allow_fp4:
            supported.discard("fp4")
        for prec in SAFE_FALLBACKS[preferred]:
            if prec == "fp4" and "fp16" not in supported:
                continue
            if prec in supported:
                return prec
        return "fp32"

    # GEMM-shaped fused forms judged by the reference's MatMul/Gemm rule.
    _GEMM_FORMS = {"MatMul": "MatMul", "Linear": "Linear", "Gemm": "Gemm", "FusedMatMulBias": "MatMul",
                   "FusedGemmEpilogue": "Gemm"}

    def executable_low_precision(self, node: Node, graph: Graph) -> Optional[str]:
        """"fp4" / "fp8" where the policy runs `node` on the W4A16 / E4M3 GEMM,
        else None: a GEMM-shaped node with a constant rank-2 weight, and the
        reference's rule's choice for it -- under "fp8" on the profile
        without fp4 (fp4 falls back to fp8), under "fp4" on this one."""
        if self.policy.name not in ("fp8", "fp4"):
            return None
        form = self._GEMM_FORMS.get(node.op_type)
        if form is None or len(node.inputs) < 2:
            return None
        w = graph.get_tensor(node.inputs[1])
        if w is None or not (w.is_initializer or w.is_constant) or len(w.shape) != 2:
            return None
        chosen = self._supported_fallback(self._preferred_tunable_precision(node, graph, form),
                                          allow_fp4=self.policy.name == "fp4")
        return chosen if chosen in ("fp8", "fp4") else None

    def executable_fp8(self, node: Node, graph: Graph) -> bool:
        """Whether the policy runs `node` on the E4M3 GEMM."""
        return self.executable_low_precision(node, graph) == "fp8"

    def _preferred_tunable_precision(self, node: Node, graph: Graph, op_type: Optional[str] = None) -> str:
        op_type = op_type or node.op_type
        if op_type in {"Conv", "Conv2d"}:
            ks = list(node.attributes.get("kernel_shape", []))
            w = graph.get_tensor(node.inputs[1]) if len(node.inputs) > 1 else None
            o = _concrete_dim(w.shape[0]) if w and w.shape else None
            c = _concrete_dim(w.shape[1]) if w and len(w.shape) > 1 else None
            aligned = o is not None and c is not None and o % 16 == 0 and c % 16 == 0
            return "fp8" if ks in ([1, 1], [1]) and aligned else "fp16"
        if op_type in {"MatMul", "Linear", "Gemm"}:
            k, n = _gemm_k_n(node, graph)
            w = graph.get_tensor(node.inputs[1]) if len(node.inputs) > 1 else None
            const_w = bool(w and (w.is_initializer or w.is_constant))
            if k is not None and n is not None:
                if const_w and k % 32 == 0 and n % 32 == 0 and k >= 128 and n >= 128 and k * n >= 32768:
                    return "fp4"
                if k % 16 == 0 and n % 16 == 0 and k >= 64 and n >= 64:
                    return "fp8"
            return "fp16"
        return "fp32"

    def get_precision_intersection(self, node: Node, graph: Graph) -> dict:
        profile = self.select_precision(node, graph)
        supported = self.hardware.supported_precisions()
        return {"node_id": node.id, "op_type": node.op_type, "selected": profile.compute_dtype,
                "supported_by_hardware": supported, "in_supported_set": profile.compute_dtype in supported,
                "profile": profile}

    # -- decomposition ------------------------------------------------------------
    def decompose(self, node: Node, graph: Graph,
                  precision: Optional[PrecisionProfile] = None) -> List[KernelSpecRef]:
        precision = precision or self.select_precision(node, graph)
        if precision.compute_dtype not in self.hardware.supported_precisions():
            raise ValueError(f"Node '{node.id}' requested unsupported precision '{precision.compute_dtype}'")
        if node.op_type in SENSITIVE_OPS and precision.compute_dtype != "fp32":
            raise ValueError(f"Sensitive operator '{node.op_type}' must decompose in fp32")
        fn = DECOMPOSE_DISPATCH.get(node.op_type)
        if fn is None:
            kernels = [KernelSpecRef(kernel_name=f"{node.op_type.lower()}_{precision.compute_dtype}",
                                     inputs=list(node.inputs), outputs=list(node.outputs),
                                     operator_params=dict(node.attributes))]
        elif node.op_type in {"Conv", "Conv2d"}:
            kernels = fn(node, graph, precision,
                         use_winograd="winograd" in self.hardware.conv_strategies_available())
        else:
            kernels = fn(node, graph, precision)
        for k in kernels:
            k.precision_profile = precision
        self.validate_decomposition(node, kernels)
        return kernels

    @staticmethod
    def validate_decomposition(node: Node, kernels: List[KernelSpecRef]) -> None:
        """Every step consumes available tensors, produces once, covers outputs."""
        if not kernels:
            raise ValueError(f"Node '{node.id}' decomposed to an empty sequence")
        available = {n for n in node.inputs if n}
        produced: Set[str] = set()
        for i, k in enumerate(kernels):
            if not k.kernel_name:
                raise ValueError(f"Node '{node.id}' kernel {i} has an empty name")
            missing = [n for n in k.inputs if n and n not in available]
            if missing:
                raise ValueError(f"Node '{node.id}' kernel '{k.kernel_name}' consumes unresolved tensors {missing}")
            outs = [n for n in k.outputs if n]
            if not outs:
                raise ValueError(f"Node '{node.id}' kernel '{k.kernel_name}' has no output")
            dup = [n for n in outs if n in produced]
            if dup:
                raise ValueError(f"Node '{node.id}' produces tensors more than once: {dup}")
            produced.update(outs)
            available.update(outs)
        missing_out = [n for n in node.outputs if n and n not in produced]
        if missing_out:
            raise ValueError(f"Node '{node.id}' lowering does not produce outputs {missing_out}")

    # -- tuning (reference formulas, c32/strategy.py:262-341) -------------------------
    def tune_kernel(self, ref: KernelSpecRef, precision: PrecisionProfile,
                    problem_size: Optional[Any] = None) -> KernelTuningParams:
        if isinstance(problem_size, ProblemSize):
            ps: Dict[str, int] = {"m": problem_size.m, "n": problem_size.n, "k": problem_size.k,
                                  "batch": problem_size.batch, "num_heads": problem_size.num_heads,
                                  "seq_len": problem_size.seq_len, **problem_size.spatial}
        else:
            ps = dict(problem_size or {})
        hw = self.hardware
        max_threads, max_smem = hw.max_threads_per_block, hw.smem_bytes
        max_bx, max_grid = min(max_threads, hw.max_block_dim), hw.max_grid_dim
        name = ref.kernel_name
        if name.startswith("matmul_"):
            m, n, k = ps.get("m", 1024), ps.get("n", 1024), ps.get("k", 1024)
            bx = min(128, max_bx)
            by = min(8, max(1, max_threads // max(1, bx)))
            dbytes = 2 if precision.input_dtype in {"fp16", "bf16"} else 4
            smem = (bx + by) * min(max(1, k), 32) * dbytes
            return KernelTuningParams(block_x=bx, block_y=by, grid_x=_clamp_grid(_ceil_div(max(1, n), bx), max_grid),
                                      grid_y=_clamp_grid(_ceil_div(max(1, m), by), max_grid),
                                      smem_bytes=_clamp_smem(smem, max_smem))
        if name.startswith("winograd_forward_"):
            return KernelTuningParams(block_x=min(256, max_bx),
                                      grid_x=_clamp_grid(max(1, ps.get("out_channels", 64)), max_grid),
                                      smem_bytes=_clamp_smem(ps.get("smem", 16384), max_smem))
        if name.startswith("im2col_"):
            bx = min(256, max_bx)
            return KernelTuningParams(block_x=bx, grid_x=_clamp_grid(_ceil_div(max(1, ps.get("num_tiles", 4096)), bx),
                                                                     max_grid))
        if name.startswith(("reduce_", "exp", "sqrt")) or any(
                name.startswith(p) for p in ("add_", "mul_", "div_", "sub_", "relu_", "erf_", "add_bias_")):
            bx = min(256, max_bx)
            return KernelTuningParams(block_x=bx, grid_x=_clamp_grid(_ceil_div(max(1, ps.get("elements", 1024)), bx),
                                                                     max_grid))
        if name in ("reshape", "transpose", "flatten", "split", "gather", "constant", "squeeze"):
            bx = min(128, max_bx)
            return KernelTuningParams(block_x=bx, grid_x=_clamp_grid(_ceil_div(max(1, ps.get("elements", 1024)), bx),
                                                                     max_grid))
        return KernelTuningParams(block_x=min(128, max_bx), grid_x=1)

    def process_graph(self, graph: Graph) -> Dict[str, Any]:
        if not graph.node_order:
            graph.topological_sort()
        results = {}
        for nid in graph.node_order:
            node = graph.nodes[nid]
            precision = self.select_precision(node, graph)
            kernels = self.decompose(node, graph, precision)
            for k in kernels:
                k.tuning_params = self.tune_kernel(k, precision)
            results[nid] = {"node": node, "precision": precision, "kernels": kernels}
        return results

    def _is_kernel_tunable(self, name: str) -> bool:
        return name not in METADATA_KERNELS


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def _concrete_dim(value: Any) -> Optional[int]:
    try:
        v = int(value)
    except (TypeError, ValueError):
        return None
    return v if v > 0 else None


def _gemm_k_n(node: Node, graph: Graph):
    if len(node.inputs) < 2:
        return None, None
    a, b = graph.get_tensor(node.inputs[0]), graph.get_tensor(node.inputs[1])
    if a is None or b is None or len(a.shape) < 2 or len(b.shape) < 2:
        return None, None
    k = _concrete_dim(a.shape[-2] if int(node.attributes.get("transA", 0)) else a.shape[-1])
    n = _concrete_dim(b.shape[-2] if int(node.attributes.get("transB", 0)) else b.shape[-1])
    return k, n


def _clamp_smem(smem: int, max_smem: int) -> int:
    if smem == -1:
        return -1
    if smem < 0:
        return 0
    return -1 if smem > max_smem else smem


def _clamp_grid(grid: int, max_grid: int) -> int:
    return min(max(1, int(grid)), max_grid)
