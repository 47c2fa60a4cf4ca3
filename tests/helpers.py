"""Shared helpers of the parity tests: seeded inputs, paired oracle / device
blocks with identical initial state, and the error metrics the tests gate on.

Metrics (both are reported by every check):
  normwise(a, r)    = max|a - r| / max|r|
  elementwise(a, r) = max over elements of |a - r| / max(|r|, 1e-3 rms(r))

Gates (north star): fp32 paths within 1e-4 of the fp32 oracle, taken
element by element (elementwise <= 1e-4, which implies normwise <= 1e-4);
fp16 paths within 2e-2 normwise of the fp32 oracle.  The floor 1e-3 rms(r)
keeps outputs that are exactly or nearly zero (a ReLU's dead units, a sum of
terms that cancel) from turning the relative error into a division by zero.

Every check appends (test, name, normwise, elementwise, gate) to RECORDS;
tests/conftest.py writes them to the file named by SOKLYN_PARITY_REPORT.
"""
from __future__ import annotations

import os

import numpy as np

FP32_TOL = 1e-4   # north star: fp32 paths within 1e-4 relative of the reference's fp32 results
FP16_TOL = 2e-2   # north star: fp16 paths within 2e-2 relative of an fp32 reference
RMS_FLOOR = 1e-3  # elementwise metric: denominator floor as a fraction of rms(r)

RECORDS: list[dict] = []


def normwise(a, r) -> float:
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    den = np.max(np.abs(r)) if r.size else 0.0
    if a.size == 0:
        return 0.0
    if den == 0:
        return float(np.max(np.abs(a)))
    return float(np.max(np.abs(a - r)) / den)


def elementwise(a, r) -> float:
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    if a.size == 0:
        return 0.0
    floor = RMS_FLOOR * float(np.sqrt(np.mean(r * r)))
    den = np.maximum(np.abs(r), floor)
    diff = np.abs(a - r)
    if floor == 0:
        # r is all zeros: absolute error
        return float(np.max(diff))
    return float(np.max(diff / den))


def check(name, a, r, tol) -> float:
    """Compare a device result with the oracle's.  tol <= FP32_TOL gates the
    elementwise metric (fp32 paths); a looser tol gates the normwise metric
    (fp16 paths).  Returns the gated value."""
    a = np.asarray(a)
    r = np.asarray(r)
    assert a.shape == r.shape, f"{name}: shape {a.shape} != {r.shape}"
    nw = normwise(a, r)
    ew = elementwise(a, r)
    gate = "elementwise" if tol <= FP32_TOL else "normwise"
    val = ew if gate == "elementwise" else nw
    RECORDS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "name": name,
                    "normwise": nw, "elementwise": ew, "gate": gate, "tol": tol})
    print(f"  {name}: normwise {nw:.2e}  elementwise {ew:.2e}  (gate {gate} <= {tol:.0e})", flush=True)
    assert val <= tol, f"{name}: {gate} error {val:.3e} > {tol:.1e} (normwise {nw:.3e}, elementwise {ew:.3e})"
    return val


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def he_normal(g: np.random.Generator, fan_in: int, fan_out: int) -> np.ndarray:
    return (g.standard_normal((fan_in, fan_out)) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
