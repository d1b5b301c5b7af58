"""Ahead-of-time build of libc3hip.so for gfx950.

Each HIP translation unit under ``csrc/`` is compiled to an object in
``_build/`` (in parallel) and linked into ``hackathon_amd/libc3hip.so``, the
in-tree library the ctypes binding loads.  There is no JIT anywhere on the
execution path: the reference compiled its CUDA kernels with NVRTC inside the
timed region (c35/engine.py:798-828); this build does all compilation here.

Usage:  python -m hackathon_amd.build [--jobs N]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libc3hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wno-pass-failed",
    # Compiler-formed packed fp32 ops are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libc3hip.so")
    return path


# Per-source additions.  attention.hip: MFMA accumulators in ordinary VGPRs
# (the flash kernel's softmax reads and rescales them every K tile; in AGPRs
# each access costs a v_accvgpr_read / write pair).
EXTRA_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libc3hip.so."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args()
    build(args.jobs)


if __name__ == "__main__":
    main()
