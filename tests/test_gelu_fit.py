"""The erf fit behind the staging kernels' erf-GELU (sam.cpp_amd/csrc/q8stage.hpp
gelu_erf), replayed on the CPU in float32.

The device evaluates erf(t) = sign(t) (1 - r exp(-a^2) P(r - 1)), a = min(|t|, 4),
r = 1 / (1 + 0.55 a), with a degree-7 P, then GELU = 0.5 v (1 + erf(v / sqrt 2))
as ggml_gelu_erf orders it.  Here every step is rounded to float32 as the GPU
rounds it: fma through float64 then one rounding, a correctly rounded reciprocal
and exp2 (the hardware's are within 1 ulp of those).  The coefficients are read
from the header, so a slipped digit there fails the error bound.
"""

import math
import os
import re
import sys

import numpy as np
import pytest
from scipy import special

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sam.cpp_amd", "csrc",
                      "q8stage.hpp")
F = np.float32


def _coefficients():
    text = open(HEADER).read()
    body = text[text.index("float gelu_erf(float v)"):]
    body = body[:body.index("\n}\n")]
    first = re.search(r"float p = (-?[0-9.]+)f;", body).group(1)
    rest = re.findall(r"p = __builtin_fmaf\(p, u, (-?[0-9.]+)f\);", body)
    slope = re.search(r"__builtin_fmaf\(a, ([0-9.]+)f, 1\.f\)", body).group(1)
    clamp = re.search(r"fminf\(fabsf\(t\), ([0-9.]+)f\)", body).group(1)
    return [float(first)] + [float(c) for c in rest], float(slope), float(clamp)


def _fma(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F)


def _erfc_fit(a):
    coeffs, slope, _ = _coefficients()
    r = (1.0 / _fma(a, np.full_like(a, slope), np.ones_like(a)).astype(np.float64)).astype(F)
    u = (r - F(1)).astype(F)
    p = np.full_like(u, F(coeffs[0]))
    for c in coeffs[1:]:
        p = _fma(p, u, np.full_like(u, F(c)))
    g = np.exp2((a * a).astype(F).astype(np.float64) * np.float64(F(-1.4426950408889634))).astype(F)
    return ((r * g).astype(F) * p).astype(F)


def _erf_fit(t):
    _, _, clamp = _coefficients()
    t = np.asarray(t, F)
    a = np.fmin(np.abs(t), F(clamp))                      # fminf: NaN -> the clamp
    return np.copysign((F(1) - _erfc_fit(a)).astype(F), t)


def _gelu_fit(v):
    v = np.asarray(v, F)
    t = (v * F(0.70710678118654752440)).astype(F)
    return (F(0.5) * v * (F(1) + _erf_fit(t))).astype(F)


def test_coefficients_parse():
    coeffs, slope, clamp = _coefficients()
    assert len(coeffs) == 8 and coeffs[-1] == 1.0
    assert slope == 0.55 and clamp == 4.0


def test_erf_fit_error_bound():
    """Within 2.7e-7 of erf on a dense grid over [-8, 8] (the clamp at 4
    included), exactly +-1 at +-inf; a NaN input gives the clamp's +-1 and a
    NaN GELU."""
    t = np.linspace(-8.0, 8.0, 2_000_001).astype(F)
    t = np.concatenate([t, np.float32([0.0, -0.0, 1e-30, -1e-30, 3.9999998, 4.0, 4.0000005])])
    err = np.abs(_erf_fit(t).astype(np.float64) - special.erf(t.astype(np.float64)))
    assert err.max() <= 2.7e-7, (err.max(), t[err.argmax()])
    # where 1 + erf is small (a >= 2) the erfc term itself is within a few
    # 1e-9 (what remains is the float32 rounding of 1 - erfc)
    a = np.linspace(2.0, 4.0, 200_001).astype(F)
    assert np.abs(_erfc_fit(a).astype(np.float64) - special.erfc(a.astype(np.float64))).max() <= 3e-9
    assert _erf_fit(np.float32([np.inf]))[0] == 1.0 and _erf_fit(np.float32([-np.inf]))[0] == -1.0
    assert abs(_erf_fit(np.float32([np.nan]))[0]) == 1.0
    assert np.isnan(_gelu_fit(np.float32([np.nan]))[0])


def test_gelu_zero_below_clamp():
    """Past a = 4 (t <= -4, v <= -4 sqrt 2) 1 - erfc(4) rounds to 1 in float32,
    so the GELU is exactly 0 there (ggml's erff gives -1 there as well)."""
    v = -np.linspace(4 * math.sqrt(2), 60.0, 10001).astype(F)
    v = v[v * F(0.70710678118654752440) <= F(-4)]
    assert v.size > 9000
    g = _gelu_fit(v)
    assert np.all(g == 0.0)


def test_gelu_fit_matches_exact_gelu():
    """Against 0.5 v (1 + erf(v / sqrt 2)) in float64, on N(0, 1)-like inputs:
    the absolute error is at most 0.5 |v| 2.7e-7 plus float32 rounding."""
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(200_000), rng.uniform(-12, 12, 200_000)]).astype(F)
    exact = 0.5 * v.astype(np.float64) * (1.0 + special.erf(v.astype(np.float64) / math.sqrt(2.0)))
    got = _gelu_fit(v).astype(np.float64)
    bound = 0.5 * np.abs(v) * 2.7e-7 + 2.0 * np.abs(exact) * 2.0 ** -24 + 1e-45
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("slip", [1e-4, -1e-4])
def test_a_slipped_coefficient_breaks_the_bound(slip, monkeypatch):
    """The bound is tight enough to catch a coefficient off by 1e-4."""
    coeffs, slope, clamp = _coefficients()
    bad = list(coeffs)
    bad[3] += slip
    monkeypatch.setattr(sys.modules[__name__], "_coefficients", lambda: (bad, slope, clamp))
    t = np.linspace(-4.0, 4.0, 400_001).astype(F)
    err = np.abs(_erf_fit(t).astype(np.float64) - special.erf(t.astype(np.float64)))
    assert err.max() > 2.7e-7
