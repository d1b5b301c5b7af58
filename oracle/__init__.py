"""NumPy oracle for the C3 numerical path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of
`bench.py` may import this package, and only as the checker.  The product
(`hackathon_amd/`) never imports, links or calls anything here; its kernels
fail loudly when libc3hip.so is missing instead of falling back to a CPU path.

* `registry_ref`: the C3.2 kernel registry (c32/kernel_registry.py) and the
  C3.5 fused-op semantics (c35/engine.py), plus ONNX closed forms for the ops
  the reference lacks (MaxPool, Quantize/QLinearMatMul/Dequantize, ArgMax).
* `graph_ref`: BN folding (c35/executor.py:359-442), plan-order evaluation
  (`run_plan`, with bf16/fp16 rounding emulation at node boundaries), unfused
  ONNX-semantics evaluation (`run_graph`) and W8A8 calibration ranges.

Pinning: tests/test_oracle.py checks every function here against closed
forms, brute-force loops and the reference tests' formula-generated fixtures.
"""
