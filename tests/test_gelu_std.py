"""The GELU form the GEMM epilogues use for the standard constants
(`gelu_std`, hackathon_amd/csrc/gemm_kernels.h), evaluated on the CPU as the
kernel evaluates it: the degree-8 polynomial P of log2 Phi(-a) in fp32
Horner steps (each fma rounded once), E = 2^P, erf(x / sqrt 2) =
sign(x) fl(1 - 2E), then (x (erf + 1)) 0.5.  The coefficients are read from
the header, so this pins the committed polynomial: its fit against
log2 Phi(-a) (scipy's log_ndtr), its accuracy against x Phi(x) and against
the decomposed chain with a correctly rounded erf (the bound of the GPU test
test_gemm_gelu_epilogue_matches_the_chain), and the chain's special values.
The GPU tests check the kernels against the chain; this checks the formula.
"""

from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
from scipy.special import erf, log_ndtr, ndtr

HEADER = Path(__file__).resolve().parents[1] / "hackathon_amd" / "csrc" / "gemm_kernels.h"
F = np.float32


def _coefficients():
    body = HEADER.read_text()
    m = re.search(r"float gelu_std\(float x\) \{(.*?)\n\}", body, re.S)
    assert m, "gelu_std not found"
    src = m.group(1)
    clamp = float(re.search(r"fminf\(fabsf\(x\), ([0-9.]+)f\)", src).group(1))
    first = re.search(r"float p = (-?0x[0-9a-fp.+-]+)f;", src).group(1)
    rest = re.findall(r"p = fmaf\(p, a, (-?0x[0-9a-fp.+-]+|-?[0-9.]+)f\);", src)
    hexes = [first] + rest  # highest degree first
    vals = [float.fromhex(h) if "x" in h else float(h) for h in hexes]
    return clamp, vals


def _fma32(a, b, c):
    # a * b is exact in float64 (two 24-bit significands); one rounding of the sum to fp32
    return (a.astype(np.float64) * b.astype(np.float64) + np.asarray(c, np.float64)).astype(F)


def _gelu_std(x):
    clamp, c = _coefficients()
    x = np.asarray(x, F)
    a = np.minimum(np.abs(x), F(clamp))
    p = np.full_like(a, F(c[0]))
    for ck in c[1:]:
        p = _fma32(p, a, np.full_like(a, F(ck)))
    e = np.exp2(p.astype(np.float64)).astype(F)  # v_exp_f32: within an ulp; modelled correctly rounded
    erf_q = np.copysign(_fma32(np.full_like(e, F(-2.0)), e, np.full_like(e, F(1.0))), x)
    with np.errstate(invalid="ignore"):
        return ((x * (erf_q + F(1.0))).astype(F) * F(0.5)).astype(F)


def _chain(x):
    x = np.asarray(x, F)
    q = (x / F(math.sqrt(2.0))).astype(F)
    e = erf(q.astype(np.float64)).astype(F)
    with np.errstate(invalid="ignore"):
        return ((x * (e + F(1.0))).astype(F) * F(0.5)).astype(F)


def test_coefficients_fit_log2_phi():
    """P fits log2 Phi(-a) on [0, clamp] to within 1.7e-8 of Phi(-a) itself
    (the weighted fit's bound), with P(0) = -1 exactly."""
    clamp, c = _coefficients()
    assert len(c) == 9 and c[-1] == -1.0 and all(float(F(v)) == v for v in c)
    a = np.linspace(0.0, clamp, 200001)
    got = np.exp2(np.polyval(c, a))
    want = np.exp2(log_ndtr(-a) / math.log(2.0))
    assert np.max(np.abs(got - want)) < 1.7e-8
    # at the clamp 1 - 2E rounds to 1 in fp32, as erf rounds to -1 in the chain
    assert F(1.0) - F(2.0) * F(got[-1]) == F(1.0)


def test_accuracy_against_gelu_and_the_chain():
    """Within 2 |x| 2^-24 of x Phi(x) on [-12, 12] (the chain's own roundings
    reach 1.8), and within the GPU test's bound of the chain everywhere."""
    x = np.linspace(-12.0, 12.0, 1_000_001, dtype=F)
    got = _gelu_std(x).astype(np.float64)
    exact = x.astype(np.float64) * ndtr(x.astype(np.float64))
    unit = np.abs(x.astype(np.float64)) * 2.0 ** -24 + 1e-38
    assert np.max(np.abs(got - exact) / unit) < 2.0
    ref = _chain(x).astype(np.float64)
    tol = 2.0 ** -21 * np.abs(ref) + np.abs(x.astype(np.float64)) * 2.0 ** -22 + 1e-38
    assert np.max(np.abs(got - ref) / tol) < 0.5


def test_special_values_are_the_chains():
    x = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-8, -1e-8, -5.6, -8.0, -30.0, np.inf, -np.inf, np.nan], F)
    got, ref = _gelu_std(x), _chain(x)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got[fin], ref[fin])          # values, including +Inf
    np.testing.assert_array_equal(np.signbit(got[fin]), np.signbit(ref[fin]))  # -0 where the chain gives -0
