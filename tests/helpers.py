"""Shared test helpers: seeded inputs from the reference's own generator (Philox4x32-10 via the
oracle), the reference tests' quarter-integer generator, and the parity measures of the
north-star bar (max relative error 1e-5*sqrt(K) against a magnitude scale)."""
from __future__ import annotations

import math

import numpy as np


def quarter_input(n: int, seed: int) -> np.ndarray:
    """Multiples of 0.25 in [-4, 4] from the LCG of the reference's matmul tests
    (tests/ops/matmul_test.cpp:26-35). Products are multiples of 1/16 with |p| <= 16, so any
    sum of up to 2^20 of them is exact in fp32 in any order."""
    out = np.empty(n, dtype=np.float32)
    state = seed & 0xFFFFFFFF
    # vectorised form of state = state*1664525 + 1013904223 (mod 2^32)
    vals = np.empty(n, dtype=np.uint64)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        vals[i] = state
    out[:] = (((vals >> 12).astype(np.int64) % 33) - 16).astype(np.float32) / 4
    return out


def quarter_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """Large quarter-integer matrices (the LCG above is too slow in Python for millions of
    entries): multiples of 0.25 in [-4, 4] from numpy's generator."""
    rng = np.random.default_rng(seed)
    return (rng.integers(-16, 17, size=(rows, cols)).astype(np.float32) / 4).astype(np.float32)


def uniform(oracle, shape, low, high, seed, offset=0) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    return oracle.uniform(n, low, high, seed, offset).reshape(shape)


def normal(oracle, shape, mean, std, seed, offset=0) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    return oracle.normal(n, mean, std, seed, offset).reshape(shape)


def tolerance(k: int) -> float:
    """The north-star parity bar: max relative error 1e-5 * sqrt(K)."""
    return 1e-5 * math.sqrt(max(k, 1))


def gemm_errors(got, want, scale):
    """(max |got-want| / scale_i, max |got-want| / max|want|): error relative to the per-entry
    magnitude sum_p |a*b| (tests/reference/blas.hpp:38-59) and to the largest entry."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    rel_mag = float(np.max(err / (np.asarray(scale, dtype=np.float64) + 1e-30))) if err.size else 0.0
    top = float(np.max(np.abs(want))) if want.size else 0.0
    rel_max = float(np.max(err) / top) if top > 0 else float(np.max(err) if err.size else 0.0)
    return rel_mag, rel_max


def assert_gemm_parity(got, want, scale, k, what=""):
    rel_mag, rel_max = gemm_errors(got, want, scale)
    bar = tolerance(k)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert rel_mag <= bar and rel_max <= bar, (
        f"{what}: rel err vs magnitude {rel_mag:.3e}, vs max|C| {rel_max:.3e}, bar {bar:.3e}")
    return rel_mag, rel_max


def magnitude(oracle, a, b) -> np.ndarray:
    """sum_p |a_ip * b_pj| for every entry, via the oracle's fp32 product of |A| and |B| (a scale
    for the error bound, so its own rounding does not matter)."""
    return oracle.matmul(np.abs(a), np.abs(b)).astype(np.float64)


def same_elements(x, y) -> np.ndarray:
    """Elementwise bit equality of two float32 arrays of one shape."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    return x.view(np.uint32) == y.view(np.uint32)


def same_bits(x, y) -> bool:
    x = np.ascontiguousarray(x)
    y = np.ascontiguousarray(y)
    return x.shape == y.shape and x.dtype == y.dtype and bool(
        np.all(x.view(np.uint8) == y.view(np.uint8)))


def record_parity(case: str, **fields) -> None:
    """Adds `case`'s measured parity figures to gpurun_out/parity.json (or the file named by
    MFR_PARITY_JSON), merging with what earlier tests of the run wrote, so the figures behind the
    pass/fail verdicts are kept, not only printed."""
    import json
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    path = os.environ.get("MFR_PARITY_JSON", os.path.join(root, "gpurun_out", "parity.json"))
    os.makedirs(os.path.dirname(path), exist_ok=True)
    data = {}
    if os.path.exists(path):
        try:
            with open(path) as fh:
                data = json.load(fh)
        except ValueError:
            data = {}
    data[case] = {k: (float(v) if isinstance(v, (np.floating, float)) else
                      int(v) if isinstance(v, (np.integer, int)) and not isinstance(v, bool) else v)
                  for k, v in fields.items()}
    tmp = path + ".tmp"
    with open(tmp, "w") as fh:
        json.dump(data, fh, indent=1, sort_keys=True)
    os.replace(tmp, path)
