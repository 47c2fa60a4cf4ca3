"""Shared helpers of the parity tests: seeded inputs, paired oracle / device
blocks with identical initial state, and the error metrics the tests gate on.

Metrics:
  normwise(a, r) = max|a - r| / max|r|          (gate: fp32 1e-4, fp16 2e-2)
"""
from __future__ import annotations

import numpy as np

FP32_TOL = 1e-4   # north star: fp32 paths within 1e-4 relative of the reference's fp32 results
FP16_TOL = 2e-2   # north star: fp16 paths within 2e-2 relative of an fp32 reference


def normwise(a, r) -> float:
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    den = np.max(np.abs(r))
    if den == 0:
        return float(np.max(np.abs(a)))
    return float(np.max(np.abs(a - r)) / den)


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def he_normal(g: np.random.Generator, fan_in: int, fan_out: int) -> np.ndarray:
    return (g.standard_normal((fan_in, fan_out)) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
