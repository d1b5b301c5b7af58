"""CPU oracle of the W4A16 precision (MXFP4 weights, fp16 activations) (NumPy).

TEST INFRASTRUCTURE ONLY (see oracle/registry_ref.py).

The reference chooses fp4 for large aligned constant-weight GEMMs
(c32/strategy.py:150-154) and runs it as W4A16: activations stay fp16,
constant weights are fp4, accumulation and output fp32 (c32/strategy.py:
101-108).  It declares this structurally only (docs/remaining-problems.md:34)
and fixes no number format.  This module fixes the one the HIP path
implements, the OCP Microscaling (MX) v1.0 FP4 format:

* Element: E2M1 -- sign, 2 exponent bits (bias 1), 1 mantissa bit; the
  magnitudes of codes 0..7 are 0, 0.5, 1, 1.5, 2, 3, 4, 6 (MX v1.0 table of
  FP4 E2M1 values); bit 3 is the sign.  No Inf or NaN codes.
* Block: 32 consecutive elements along K share an E8M0 scale, a biased
  power-of-two exponent byte (0xFF is NaN).
* Quantization of a block x[0..31] (float32): amax = max |x|;
  e = clamp(floor(log2 amax) - 2, -13, 13) (-13 for amax = 0): the MX
  shared-exponent rule floor(log2 amax) - emax(E2M1) with emax = 2, limited
  so that every dequantized element is zero or a normal fp16 (0.5 * 2^-13 =
  2^-14 .. 6 * 2^13 = 49152) and therefore exactly the fp16 value the
  W4A16 GEMM multiplies; the scale byte is e + 127.  Elements:
  E2M1(|x| * 2^-e) rounded to the nearest magnitude, ties to the even code,
  saturating at 6; the sign bit is set for negative x unless the magnitude
  code is 0.  A block holding Inf or NaN gets scale 0xFF and zero codes.
  Codes pack two per byte, element 2j in the low nibble.
* GEMM: out[m, n] = sum_k A[m, k] * W[n, k] with A in fp16 and
  W = dequantize(codes, scales) -- every product exact in fp32 and the sum
  in float64 here; the GPU accumulates in fp32 on the fp16 MFMA, so the
  comparison is to fp32 accumulation tolerance (and bit for bit against the
  fp16 GEMM on the dequantized weights).

The encoder here picks the nearest magnitude by exhaustive search over the 8
magnitudes (ties to the even code); the GPU kernel compares against the
rounding boundaries -- two different constructions of the same rounding.

Pinned (tests/test_oracle_fp4.py): `decode` against the MX v1.0 table;
`encode` against every magnitude, every midpoint (the tie direction fixed by
the even code), saturation and a dense sweep checked by the error bound
|m - decode(encode(m))| <= half the local code spacing; `quantize_mxfp4`
against the format's invariants (scaled amax in [4, 8) for unclamped blocks,
the clamp range, exact round trips of representable blocks, Inf/NaN
blocks); `gemm_w4a16` against a plain float64 matmul of integer-valued
operands.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np

F32 = np.float32
BLOCK = 32
E_MIN, E_MAX = -13, 13
NAN_SCALE = 0xFF
# |E2M1| of codes 0..7 (OCP MX v1.0, FP4 E2M1).
MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float64)


def decode(codes: np.ndarray) -> np.ndarray:
    """E2M1 codes (0..15, any integer dtype) -> float32 values."""
    c = np.asarray(codes).astype(np.int64)
    mag = MAGNITUDES[c & 7]
    return np.where(c & 8, -mag, mag).astype(F32)


def encode(m: np.ndarray) -> np.ndarray:
    """|value| (float, >= 0) -> magnitude code 0..7: nearest magnitude, ties to
    the even code, saturating at 6.  Exhaustive search over the 8 magnitudes."""
    m = np.asarray(m, np.float64)
    dist = np.abs(m[..., None] - MAGNITUDES)                 # [..., 8]
    best = dist.min(axis=-1, keepdims=True)
    cand = dist == best
    # among the (at most two) nearest codes prefer the even one
    even = cand & (np.arange(8) % 2 == 0)
    code = np.where(even.any(axis=-1), even.argmax(axis=-1), cand.argmax(axis=-1))
    return np.where(m > 6.0, 7, code).astype(np.uint8)


def block_exponent(amax: np.ndarray) -> np.ndarray:
    """Shared exponent e of blocks with the given amax (finite, >= 0)."""
    amax = np.asarray(amax, np.float64)
    out = np.full(amax.shape, E_MIN, np.int64)
    pos = amax > 0
    # floor(log2 amax) from the float's own exponent (exact, subnormals too)
    _, ex = np.frexp(amax[pos])
    out[pos] = np.clip(ex.astype(np.int64) - 1 - 2, E_MIN, E_MAX)
    return out


def quantize_mxfp4(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """x [rows, cols] (cols % 32 == 0) -> (codes [rows, cols/2] uint8,
    scales [rows, cols/32] uint8)."""
    x = np.asarray(x, F32)
    rows, cols = x.shape
    assert cols % BLOCK == 0
    xb = x.reshape(rows, cols // BLOCK, BLOCK)
    bad = ~np.isfinite(xb).all(axis=-1)
    amax = np.where(bad, 0.0, np.abs(np.where(np.isfinite(xb), xb, 0.0)).max(axis=-1))
    e = block_exponent(amax)
    inv = np.exp2(-e.astype(np.float64)).astype(F32)        # exact powers of two
    scaled = (np.abs(xb) * inv[..., None]).astype(F32)      # fp32 product, as on the GPU
    mag = encode(np.where(np.isfinite(scaled), scaled, 0.0))
    code = np.where((mag != 0) & (xb < 0), mag | 8, mag).astype(np.uint8)
    code = np.where(bad[..., None], 0, code).astype(np.uint8)
    flat = code.reshape(rows, cols)
    packed = (flat[:, 0::2] | (flat[:, 1::2] << 4)).astype(np.uint8)
    scales = np.where(bad, NAN_SCALE, e + 127).astype(np.uint8)
    return packed, scales


def unpack(codes: np.ndarray) -> np.ndarray:
    """[rows, cols/2] packed bytes -> [rows, cols] codes (element 2j low nibble)."""
    c = np.asarray(codes, np.uint8)
    out = np.empty((c.shape[0], c.shape[1] * 2), np.uint8)
    out[:, 0::2] = c & 0xF
    out[:, 1::2] = c >> 4
    return out


def dequantize_mxfp4(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(codes [rows, cols/2], scales [rows, cols/32]) -> float32 [rows, cols]."""
    vals = decode(unpack(codes)).astype(np.float64)
    rows, cols = vals.shape
    s = np.asarray(scales, np.uint8).astype(np.float64)
    sc = np.where(s == NAN_SCALE, np.nan, np.exp2(s - 127.0))
    return (vals.reshape(rows, cols // BLOCK, BLOCK) * sc[..., None]).reshape(rows, cols).astype(F32)


def gemm_w4a16(a: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """sum_k fp16(A)[m, k] * W[n, k] in float64 (W from the MXFP4 operand)."""
    a16 = np.asarray(a, np.float32).astype(np.float16).astype(np.float64)
    w = dequantize_mxfp4(codes, scales).astype(np.float64)
    return a16 @ w.T
