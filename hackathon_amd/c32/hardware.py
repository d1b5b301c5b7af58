"""Hardware capability snapshot (counterpart of c32/hardware.py).

The reference builds its snapshot from CUDA device properties
(c32/hardware.py:97-163).  Here the snapshot comes from libc3hip.so's
`c3h_device_props` on the GPU, or from the MI355X datasheet when no device is
visible (planning runs on the CPU; nothing on the CPU executes kernels).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Set, Tuple


@dataclass
class HardwareCapability:
    name: str = "AMD Instinct MI355X (gfx950, datasheet)"
    source: str = "datasheet"
    verified: bool = False
    compute_capability: Optional[Tuple[int, int]] = (9, 5)
    arch: str = "gfx950"
    compute_units: int = 256
    wavefront_size: int = 64
    max_threads_per_block: int = 1024
    max_block_dim: int = 1024
    max_grid_dim: int = 2147483647
    smem_bytes: int = 160 * 1024
    max_shared_memory_per_block: int = 160 * 1024
    smem_bytes_total: int = 256 * 160 * 1024
    hbm_bytes: int = 288 * 1024 ** 3
    supports_fp16: bool = True
    supports_bf16: bool = True
    supports_fp8: bool = True
    # CDNA4 decodes MXFP4 (E2M1 + E8M0 block exponents) natively; "fp4" is run
    # as W4A16 (c32/strategy.py:101-108) by c3h_gemm_w4a16.
    supports_fp4: bool = True
    supports_int8: bool = True
    supports_winograd: bool = True
    extra_gemm_kernels: Set[str] = field(default_factory=set)

    def supported_precisions(self) -> List[str]:
        out = ["fp32"]
        if self.supports_fp16:
            out.append("fp16")
        if self.supports_bf16:
            out.append("bf16")
        if self.supports_fp8:
            out.append("fp8")
        if self.supports_fp4:
            out.append("fp4")
        if self.supports_int8:
            out.append("int8")
        return out

    def gemm_kernels_available(self) -> Set[str]:
        names = {f"matmul_{p.replace('fp', 'f')}" for p in self.supported_precisions()}
        return names | set(self.extra_gemm_kernels)

    def conv_strategies_available(self) -> List[str]:
        out = ["im2col", "implicit_gemm"]
        if self.supports_winograd:
            out.append("winograd")
        return out

    @classmethod
    def from_device(cls, device: int = 0) -> "HardwareCapability":
        """Query the live device through libc3hip.so."""
        from ..device import device_props

        props = device_props(device)
        lds = int(props.lds_bytes_per_block)
        arch = props.arch.decode("utf-8", "replace")
        return cls(
            name=props.name.decode("utf-8", "replace"),
            source="c3h_device_props",
            verified=True,
            compute_capability=(int(props.major), int(props.minor)),
            arch=arch,
            supports_fp4=arch.startswith("gfx950"),
            compute_units=int(props.compute_units),
            wavefront_size=int(props.warp_size),
            max_threads_per_block=int(props.max_threads_per_block),
            max_block_dim=int(props.max_block_dim_x),
            max_grid_dim=int(props.max_grid_dim_x),
            smem_bytes=lds,
            max_shared_memory_per_block=lds,
            smem_bytes_total=lds * int(props.compute_units),
            hbm_bytes=int(props.total_memory_bytes),
        )


_HARDWARE = HardwareCapability()


def get_hardware() -> HardwareCapability:
    return _HARDWARE


def set_hardware(hw: HardwareCapability) -> None:
    global _HARDWARE
    _HARDWARE = hw


def activate_device_hardware(device: int = 0) -> HardwareCapability:
    """Replace the datasheet snapshot with the live device's properties."""
    hw = HardwareCapability.from_device(device)
    set_hardware(hw)
    return hw
