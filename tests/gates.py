"""Parity gates shared by the GPU tests (pure NumPy; no GPU, no oracle imports).

north_star's gates: bit-exact int8 accumulators, gathers and argmax; rtol
1e-3 for fp32; max-abs 2e-2 on logits for bf16/fp16 with >= 99.9 % argmax
agreement.  Random-init logits are often nearly tied, so argmax agreement is
asserted where it is decidable: on every row whose fp32 top-1 / top-2 margin
exceeds twice the logits' error bound, a bound-respecting result cannot move
the argmax, and agreement there must be exact.
"""

from __future__ import annotations

import math

import numpy as np


def ulp_at(x: float, kind: str) -> float:
    """One ulp of a bf16 / fp16 value of magnitude x (x at least the smallest normal)."""
    return 2.0 ** (math.floor(math.log2(max(x, 1e-30))) - (7 if kind == "bf16" else 10))


def agree(got: np.ndarray, ref: np.ndarray) -> float:
    """Share of rows (over the last axis) whose argmax is the same."""
    g = got.reshape(-1, got.shape[-1])
    r = ref.reshape(-1, ref.shape[-1])
    return float(np.mean(np.argmax(g, -1) == np.argmax(r, -1)))


def margin_agreement(got: np.ndarray, ref32: np.ndarray, bound: float):
    """(argmax agreement on rows whose fp32 top-1 / top-2 margin exceeds 2 * bound,
    share of rows that clear it)."""
    r = ref32.reshape(-1, ref32.shape[-1]).astype(np.float64)
    g = got.reshape(-1, got.shape[-1])
    top2 = np.sort(r, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2.0 * bound
    if not clear.any():
        return 1.0, 0.0
    return float(np.mean(np.argmax(g[clear], -1) == np.argmax(r[clear], -1))), float(np.mean(clear))


def rms(x) -> float:
    return float(np.sqrt(np.mean(np.square(np.asarray(x, np.float64)))))
