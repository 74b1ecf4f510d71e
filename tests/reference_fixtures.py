"""Deterministic fixtures of the reference's own quantized-matmul tests.

These reproduce the input patterns (not code) that the reference's C++ tests
generate, so the same cases can be run against the oracle and the HIP path:
  matrix_values      tests/runtime/ggml/test_quantization.cpp:34-44
  probe_weights/rhs  tools/benchmark/cpu_quantized_matmul.hpp:63-75
Shapes follow the reference naming: width = K, rows = weight rows (N),
columns = activation rows (M).
"""

import numpy as np

# tolerances used by the reference tests
DECODED_TOL = (0.025, 0.005)     # tests/runtime/ggml/test_quantization.cpp:485
NATIVE_TOL = (5e-4, 5e-5)        # tools/benchmark/cpu_quantized_matmul.hpp:212


def matrix_values(width, rows, salt):
    r = np.arange(rows, dtype=np.int64)[:, None]
    c = np.arange(width, dtype=np.int64)[None, :]
    v = (((r * 17 + c * 13 + salt * 7) % 101) - 50).astype(np.float32) * np.float32(0.004)
    v[(r[:, 0] % 127) == 0, :] = 0.0
    return v


def probe_weights(width, rows):
    r = np.arange(rows, dtype=np.int64)[:, None]
    i = np.arange(width, dtype=np.int64)[None, :]
    v = (((r * 17 + i * 13 + 7) % 101) - 50).astype(np.float32) * np.float32(0.007)
    v[(r[:, 0] % 31) == 0, :] = 0.0
    return v


def probe_rhs(width, columns, scenario="ordinary"):
    c = np.arange(columns, dtype=np.int64)[:, None]
    i = np.arange(width, dtype=np.int64)[None, :]
    v = (((c * 19 + i * 7 + 3) % 79) - 39).astype(np.float32) * np.float32(0.009)
    if scenario == "zero":
        v[:] = 0.0
    if columns > 1:
        v[1, :] = 0.0
    if scenario == "outlier":
        v[:, 3] = np.float32(17.1)
        v[:, 41] = np.float32(-0.0013)
    return v


def within(actual, expected, tol):
    a, r = tol
    err = np.abs(actual.astype(np.float64) - expected)
    return bool(np.all(np.isfinite(actual)) and np.all(err <= a + r * np.abs(expected))), float(err.max())


def max_row_rel_l2(actual, expected):
    """Largest per-row relative L2 error (rows = activation rows)."""
    actual = actual.astype(np.float64)
    expected = expected.astype(np.float64)
    num = np.sqrt(((actual - expected) ** 2).sum(axis=1))
    den = np.sqrt((expected ** 2).sum(axis=1))
    den = np.where(den == 0, 1.0, den)
    return float((num / den).max())
