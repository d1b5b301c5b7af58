"""A BASELINE workload, built and compiled for the GPU the way it is measured.

`compile_workload` is the one route from a model to a `CompiledPlan`: the
c33 pass pipeline, the executor's Conv+BN fold (c35/executor.py:359-442,
done on the device), the c34 plan at the model's batch and precision policy,
then the compiled program with its hipGraph and concurrent launch pairs.
`bench.py` times exactly what this returns, and the full-size parity tests
compare exactly that against the oracle.
"""

from __future__ import annotations

from typing import Any, Optional, Tuple

from . import models


def compile_workload(name: str, model: Optional[models.Model] = None, use_graph: bool = True,
                     concurrent: bool = True, keep_values: bool = False,
                     **build_kw: Any) -> Tuple[models.Model, Any, Any]:
    """(model, plan, CompiledPlan) for a workload of `models.CONFIGS`.

    `model` may be passed pre-built (its graph is fused in place); otherwise
    `models.build(name, **build_kw)` makes it at the BASELINE size unless
    `build_kw` overrides a dimension.  `keep_values` gives every stored
    value memory of its own so that tests can read intermediates back.
    """
    from .c32.strategy import PrecisionPolicy
    from .c33.pipeline import GraphPassPipeline
    from .c34.scheduler import ExecutionScheduler
    from .c35.compiled import CompiledPlan
    from .c35.executor import fold_conv_batchnorm, load_weights

    m = model if model is not None else models.build(name, **build_kw)
    GraphPassPipeline().run(m.graph)
    host_w, host_c = load_weights(m.weights)
    host_w.update(fold_conv_batchnorm(m.graph, host_w))
    batch = next(iter(m.inputs.values())).shape[0]
    plan = ExecutionScheduler(m.graph, batch_size=batch, precision_policy=PrecisionPolicy(m.precision)).build()
    prog = CompiledPlan(m.graph, plan, host_w, host_c, policy=m.precision, use_graph=use_graph,
                        concurrent=concurrent, keep_values=keep_values)
    return m, plan, prog
