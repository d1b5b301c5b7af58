"""CPU oracle of the fp8 (OCP E4M3) precision policy (NumPy).

TEST INFRASTRUCTURE ONLY (see oracle/registry_ref.py).

The reference declares fp8 structurally -- `matmul_f8` in the kernel
inventory (c32/hardware.py:80-81) and the mixed-precision choice of fp8 for
aligned GEMMs and 1x1 convs (c32/strategy.py:124-160, accumulation and output
fp32, c32/strategy.py:103-108) -- but has no executable fp8 kernel or numeric
definition (docs/remaining-problems.md:61-68).  This module fixes the numeric
definition the HIP path implements:

* Format: OCP 8-bit floating point E4M3 ("e4m3fn"): sign, 4 exponent bits
  (bias 7), 3 mantissa bits; no infinities; S.1111.111 is NaN; largest
  finite 448 = 1.75 * 2^8; subnormals m * 2^-9 (m = 1..7).
* Encoding of a float32 value: round to nearest, ties to even, saturating at
  +-448 (finite inputs never produce NaN); NaN -> 0x7F.
* Row-wise dynamic quantization (per-token activations; per-output-channel
  weights as rows of B^T [n][k]): amax = max_k |x[r, k]| in fp32;
  scale[r] = amax / 448 and inv = min(448 / amax, FLT_MAX) (each one a
  correctly rounded fp32 division), code[r, k] = E4M3(x[r, k] * inv) (fp32
  product); a zero row
  gives scale 0 and codes 0; a row holding a non-finite value gives scale NaN
  and NaN codes.
* GEMM: out[m, n] = (sum_k dec(qa[m, k]) * dec(qb[n, k])) * sa[m] * sb[n],
  then the usual epilogue; the products are exact (4-bit significands).
  The GPU instruction adds each aligned group of 8 products at 13 bits below
  the group's largest product before accumulating in fp32 (measured on
  gfx950), so it matches this float64 sum exactly when the products of a
  group span fewer than 13 bits (integer operands), and otherwise within
  7 * 2^-13 of each group's sum |a b|.

Pinned (tests/test_oracle_fp8.py): `decode` against torch.float8_e4m3fn for all
256 codes; `encode` against torch's float32 -> float8_e4m3fn conversion on a
dense sweep of |x| <= 448, against every code's own value and every midpoint
between neighbouring codes (ties to the even code); `quantize_rows` against
its invariants (scale * 448 recovers amax within an ulp, |x - dequant| is at
most half a code step); `gemm_fp8` against a plain float64 matmul for inputs
that are exactly representable (amax 448 rows of E4M3 values).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
E4M3_MAX = 448.0
NAN_CODE = 0x7F


def decode(codes: np.ndarray) -> np.ndarray:
    """E4M3 codes (uint8) -> float32 values (NaN for 0x7F / 0xFF)."""
    c = np.asarray(codes, np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10.0))
    val = np.where((c & 0x7F) == NAN_CODE, np.nan, val)
    return (sign * val).astype(F32)


def encode(x: np.ndarray) -> np.ndarray:
    """float32 -> E4M3 codes: nearest, ties to even, saturating at +-448."""
    v = np.asarray(x, F32).astype(np.float64)
    nan = np.isnan(v)
    sign = np.signbit(v)
    a = np.minimum(np.abs(np.where(nan, 0.0, v)), E4M3_MAX)
    # Exponent of the value's binade, clamped to the subnormal range: every
    # E4M3 value in binade e is a multiple of 2^(e-3); below 2^-6 the step is 2^-9.
    _, ex = np.frexp(a)                     # a = f * 2^ex, f in [0.5, 1)
    e = np.maximum(ex - 1, -6)
    q = np.rint(a / np.exp2(e - 3.0))       # exact division by a power of two; rint: ties to even
    # q in [8, 16] for normals (16 carries into the next binade), [0, 8] below 2^-6
    carry = q >= 16
    e = np.where(carry, e + 1, e)
    q = np.where(carry, 8, q)
    normal = q >= 8
    field = np.where(normal, ((e + 7) << 3) + (q.astype(np.int64) - 8), q.astype(np.int64))
    code = field.astype(np.int64) | np.where(sign, 0x80, 0)
    code = np.where(nan, NAN_CODE, code)
    return code.astype(np.uint8)


def quantize_rows(x: np.ndarray):
    """Row-wise dynamic quantization of a [rows, k] matrix -> (codes uint8, scales float32)."""
    x = np.asarray(x, F32)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    finite = np.isfinite(rows).all(axis=1)
    amax = np.where(finite, np.abs(np.where(np.isfinite(rows), rows, 0)).max(axis=1, initial=0.0), np.nan).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = (amax / F32(E4M3_MAX)).astype(F32)
        inv = np.where(amax > 0, np.minimum(F32(E4M3_MAX) / amax, np.finfo(F32).max), F32(0)).astype(F32)
        prod = (rows * inv[:, None]).astype(F32)
    codes = encode(prod)
    codes[~finite] = NAN_CODE
    scale = np.where(finite, scale, np.nan).astype(F32)
    return codes.reshape(rows.shape), scale


def dequantize_rows(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    return (decode(codes).astype(np.float64) * np.asarray(scales, np.float64)[:, None]).astype(F32)


def gemm_fp8(qa: np.ndarray, sa: np.ndarray, qb_nk: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """out[m, n] = (sum_k dec(qa) dec(qb)) * sa[m] * sb[n] in float64 (B given as [n][k])."""
    acc = decode(qa).astype(np.float64) @ decode(qb_nk).astype(np.float64).T
    return acc * np.asarray(sa, np.float64)[:, None] * np.asarray(sb, np.float64)[None, :]


def matmul_fp8_policy(a: np.ndarray, w_kn: np.ndarray) -> np.ndarray:
    """A [.., k] @ W [k, n] under the fp8 policy: both operands quantized row-wise
    (A per row, W per output column) then `gemm_fp8`; float32 result."""
    a = np.asarray(a, F32)
    lead = a.shape[:-1]
    qa, sa = quantize_rows(a.reshape(-1, a.shape[-1]))
    qb, sb = quantize_rows(np.ascontiguousarray(np.asarray(w_kn, F32).T))
    return gemm_fp8(qa, sa, qb, sb).astype(F32).reshape(lead + (w_kn.shape[-1],))
