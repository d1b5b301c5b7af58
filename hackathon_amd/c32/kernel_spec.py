"""Kernel-decomposition data structures (counterpart of c32/kernel_spec.py).

Same dataclasses and field names as the reference (c32/kernel_spec.py:10-110)
so that plans built here and plans built by the reference planner are
interchangeable.  `int8` is a valid precision (it is in the reference's
valid set as well).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional

VALID_PRECISIONS = frozenset({"fp32", "fp16", "bf16", "fp8", "fp4", "int8"})


@dataclass
class PrecisionProfile:
    compute_dtype: str = "fp32"
    accumulator_dtype: str = "fp32"
    input_dtype: str = "fp32"
    weight_dtype: Optional[str] = None
    output_dtype: str = "fp32"

    def __post_init__(self) -> None:
        for name in ("compute_dtype", "accumulator_dtype", "input_dtype", "output_dtype"):
            if getattr(self, name) not in VALID_PRECISIONS:
                raise ValueError(f"Unknown precision '{getattr(self, name)}' in {name}")
        if self.weight_dtype is not None and self.weight_dtype not in VALID_PRECISIONS:
            raise ValueError(f"Unknown precision '{self.weight_dtype}' in weight_dtype")

    def as_dict(self) -> Dict[str, Optional[str]]:
        return {"compute_dtype": self.compute_dtype, "accumulator_dtype": self.accumulator_dtype,
                "input_dtype": self.input_dtype, "weight_dtype": self.weight_dtype,
                "output_dtype": self.output_dtype}


@dataclass
class KernelTuningParams:
    block_x: int = 128
    block_y: int = 1
    block_z: int = 1
    grid_x: int = 1
    grid_y: int = 1
    grid_z: int = 1
    smem_bytes: int = 0

    def is_valid(self, max_threads: int, max_smem: int, max_block_dim: Optional[int] = None,
                 max_grid_dim: Optional[int] = None) -> bool:
        threads = self.block_x * self.block_y * self.block_z
        dims_ok = min(self.block_x, self.block_y, self.block_z, self.grid_x, self.grid_y, self.grid_z) > 0
        smem_ok = self.smem_bytes == -1 or 0 <= self.smem_bytes <= max_smem
        block_ok = max_block_dim is None or max(self.block_x, self.block_y, self.block_z) <= max_block_dim
        grid_ok = max_grid_dim is None or max(self.grid_x, self.grid_y, self.grid_z) <= max_grid_dim
        return 0 < threads <= max_threads and dims_ok and smem_ok and block_ok and grid_ok


@dataclass
class KernelSpecRef:
    kernel_name: str
    inputs: List[str] = field(default_factory=list)
    outputs: List[str] = field(default_factory=list)
    workspace_bytes: int = 0
    tuning_params: Optional[KernelTuningParams] = None
    operator_params: Dict[str, Any] = field(default_factory=dict)
    precision_profile: Optional[PrecisionProfile] = None

    @property
    def is_tunable(self) -> bool:
        return self.tuning_params is not None


@dataclass
class ProblemSize:
    m: int = 1
    n: int = 1
    k: int = 1
    batch: int = 1
    num_heads: int = 1
    seq_len: int = 1
    spatial: Dict[str, int] = field(default_factory=dict)
