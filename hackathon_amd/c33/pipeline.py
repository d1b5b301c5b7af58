"""Fusion pass pipeline (counterpart of c33/pipeline.py).

Runs the passes in the reference's PASS_ORDER (c33/pipeline.py:108-119) with
a snapshot/rollback per pass (:187-209) and reports launch/buffer counts of
the C3.2 lowering before and after (:39-102).
"""

from __future__ import annotations

import copy
from typing import Any, Dict, List

from ..c3common.ir.graph import Graph
from .fusion import (cleanup_dead_tensors, fuse_attention_scores, fuse_conv_batchnorm, fuse_conv_epilogues,
                     fuse_elementwise_chain, fuse_gemm_epilogues, fuse_layer_normalization_kernels,
                     fuse_matmul_bias, fuse_residual_norm, fuse_softmax_dropout, fuse_transpose_reshape)

PASS_ORDER = [
    ("Conv2dBatchNorm", fuse_conv_batchnorm),
    ("MatMulBias", fuse_matmul_bias),
    ("ResidualNorm", fuse_residual_norm),
    ("SoftmaxDropout", fuse_softmax_dropout),
    ("AttentionScores", fuse_attention_scores),
    ("TransposeReshape", fuse_transpose_reshape),
    ("GemmEpilogue", fuse_gemm_epilogues),
    ("ConvEpilogue", fuse_conv_epilogues),
    ("LayerNormalizationKernel", fuse_layer_normalization_kernels),
    ("EWChain", fuse_elementwise_chain),
]


def _lowering(graph: Graph):
    from ..c32.strategy import ExecutionMode, Strategy

    strategy = Strategy(mode=ExecutionMode.FULL_FP32)
    for nid in graph.node_order:
        node = graph.nodes.get(nid)
        if node is not None:
            yield node, strategy.decompose(node, graph)


def _count_launches(graph: Graph) -> int:
    """Physical launches of the C3.2 lowering (Constant steps excluded)."""
    n = sum(1 for _, kernels in _lowering(graph) for k in kernels if k.kernel_name != "constant")
    return max(n, 1)


def _count_buffers(graph: Graph) -> int:
    """Graph edge buffers plus lowering-internal intermediates."""
    inputs = {t.name for t in graph.inputs}
    outputs = {t.name for t in graph.outputs}
    buffers = 0
    for name, t in graph.tensors.items():
        if name in inputs or t.is_initializer or t.is_constant or graph.tensor_producer.get(name) is None:
            continue
        live = [c for c in graph.tensor_consumers.get(name, []) if c in graph.nodes]
        if not live and name in outputs:
            continue
        buffers += 1
    for node, kernels in _lowering(graph):
        node_outputs = {o for o in node.outputs if o}
        buffers += len({o for k in kernels for o in k.outputs if o and o not in node_outputs})
    return max(buffers, 0)


class GraphPassPipeline:
    def __init__(self, enable_fusion: bool = True, run_validation: bool = True,
                 enable_dead_cleanup: bool = True) -> None:
        self.enable_fusion = enable_fusion
        self.run_validation = run_validation
        self.enable_dead_cleanup = enable_dead_cleanup

    def run(self, graph: Graph) -> Dict[str, Any]:
        if not graph.node_order:
            graph.topological_sort()
        if not self.enable_fusion:
            n, b = _count_launches(graph), _count_buffers(graph)
            return {"Fusion": {"enabled": False, "stats": {
                "fusion_log": [], "raw_launches": n, "optimized_launches": n, "launch_reduction": 0.0,
                "raw_buffers": b, "optimized_buffers": b, "buffer_reduction": 0.0,
                "fusions_per_pattern": {}, "total_fusions": 0, "node_count_before": len(graph.nodes),
                "node_count_after": len(graph.nodes), "validation_passed": True}}}
        log: List[Dict[str, Any]] = []
        raw_launches, raw_buffers, before = _count_launches(graph), _count_buffers(graph), len(graph.nodes)
        per_pattern: Dict[str, int] = {}
        total = 0
        for name, fn in PASS_ORDER:
            snapshot = copy.deepcopy(graph)
            mark = len(log)
            try:
                n = fn(graph, log)
                if self.run_validation:
                    graph.validate()
                if n > 0:
                    per_pattern[name] = n
                    total += n
            except Exception as exc:  # roll the graph back and keep going
                graph.__dict__.clear()
                graph.__dict__.update(snapshot.__dict__)
                del log[mark:]
                log.append({"pattern": name, "status": "error", "old_node_ids": [], "new_node_id": "",
                            "removed_tensors": [], "rejection_reason": f"Pass raised exception: {exc}"})
        if self.enable_dead_cleanup:
            cleanup_dead_tensors(graph)
        try:
            graph.topological_sort()
            graph.validate()
            ok = True
        except ValueError:
            ok = False
        launches, buffers = _count_launches(graph), _count_buffers(graph)
        return {"Fusion": {"enabled": True, "stats": {
            "fusion_log": log, "raw_launches": raw_launches, "optimized_launches": launches,
            "launch_reduction": (raw_launches - launches) / max(raw_launches, 1),
            "raw_buffers": raw_buffers, "optimized_buffers": buffers,
            "buffer_reduction": (raw_buffers - buffers) / max(raw_buffers, 1),
            "fusions_per_pattern": per_pattern, "total_fusions": total, "node_count_before": before,
            "node_count_after": len(graph.nodes), "validation_passed": ok}}}
