"""Shared helpers of the parity tests: seeded inputs, paired oracle / device
blocks with identical initial state, and the error metrics the tests gate on.

Metrics (both are reported by every check):
  normwise(a, r)    = max|a - r| / max|r|
  elementwise(a, r) = max over elements of |a - r| / max(|r|, 1e-3 rms(r))

Gates (north star): fp32 paths within 1e-4 normwise of the fp32 oracle and
within FP32_EW_TOL = 1e-2 elementwise; fp16 paths within 2e-2 normwise of the
fp32 oracle (elementwise reported).  The floor 1e-3 rms(r) keeps outputs that
are exactly or nearly zero (a ReLU's dead units, a sum of terms that cancel)
from turning the relative error into a division by zero.

Why the fp32 elementwise bound is 1e-2 and not 1e-4: on a near-zero output of
a long fp32 sum, the rounding error of the summation order alone is ~1e-3 of
the floor.  The oracle sums in the reference's order (sequential k, fp32), and
it is itself 0.9e-3 to 4.7e-3 away from the exact (float64) result in this
metric at the parity-test shapes (tests/test_oracle.py::
test_reference_order_fp32_noise_exceeds_elementwise_1e4 pins that), so 1e-4
would test the order of additions rather than the result.  1e-2 still flags
any element that is wrong by more than 1e-5 rms(r); the normwise 1e-4 gate
covers every element at the scale of the output; tests/test_gpu_accuracy.py
checks that the device's fp32 GEMM outputs are at least as close to exact
arithmetic as the reference's own order, element by element.

Every check appends (test, name, normwise, elementwise, gate) to RECORDS;
tests/conftest.py writes them to the file named by SOKLYN_PARITY_REPORT.
"""
from __future__ import annotations

import os

import numpy as np

FP32_TOL = 1e-4      # north star: fp32 paths within 1e-4 relative of the reference's fp32 results
FP32_EW_TOL = 1e-2   # fp32 elementwise bound (above the reference order's own rounding noise)
FP16_TOL = 2e-2      # north star: fp16 paths within 2e-2 relative of an fp32 reference
RMS_FLOOR = 1e-3     # elementwise metric: denominator floor as a fraction of rms(r)

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
    """Compare a device result with the oracle's: normwise <= tol, and for fp32
    paths (tol <= FP32_TOL) also elementwise <= FP32_EW_TOL.  Both metrics are
    printed and recorded.  Returns the normwise error."""
    a = np.asarray(a)
    r = np.asarray(r)
    assert a.shape == r.shape, f"{name}: shape {a.shape} != {r.shape}"
    nw = normwise(a, r)
    ew = elementwise(a, r)
    fp32 = tol <= FP32_TOL
    RECORDS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "name": name,
                    "normwise": nw, "elementwise": ew, "tol": tol, "ew_tol": FP32_EW_TOL if fp32 else None})
    gates = f"normwise <= {tol:.0e}" + (f", elementwise <= {FP32_EW_TOL:.0e}" if fp32 else "")
    print(f"  {name}: normwise {nw:.2e}  elementwise {ew:.2e}  (gates: {gates})", flush=True)
    assert nw <= tol, f"{name}: normwise error {nw:.3e} > {tol:.1e} (elementwise {ew:.3e})"
    if fp32:
        assert ew <= FP32_EW_TOL, f"{name}: elementwise error {ew:.3e} > {FP32_EW_TOL:.1e} (normwise {nw:.3e})"
    return nw


def check_sum_bound(name, a, r, scale, tol=FP32_TOL) -> float:
    """fp32 GEMM outputs element by element: |a - r| <= tol * scale, where scale is the
    element's sum over k of |x_k w_k| (plus |bias|): the bound the rounding of any
    order of the k additions stays within (n u scale, u = 2^-24, far below 1e-4 for
    these k), so unlike |a - r| / |r| it does not fail on outputs that cancel to near
    zero, and unlike the normwise metric it holds for every element."""
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    scale = np.asarray(scale, np.float64)
    assert a.shape == r.shape == scale.shape, f"{name}: shapes {a.shape} {r.shape} {scale.shape}"
    worst = float(np.max(np.abs(a - r) / np.maximum(scale, np.finfo(np.float64).tiny)))
    RECORDS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "name": name + " (sum bound)",
                    "normwise": None, "elementwise": worst, "tol": tol, "ew_tol": tol})
    print(f"  {name}: max |a - r| / sum|terms| {worst:.2e}  (gate {tol:.0e} per element)", flush=True)
    assert worst <= tol, f"{name}: element error {worst:.3e} of its summation scale > {tol:.0e}"
    return worst


def check_adam_update(name, w0, w1, dm, dv, lr, step, ref_update, ref_dm, beta1=0.9, beta2=0.999, eps=1e-8):
    """The Adam step on the fp32 master (backward.cu:133-147): w1 - w0 must equal
    -lr * (dm / (1 - beta1^t)) / (sqrt(dv / (1 - beta2^t)) + eps) computed from the
    device's own moments (to f32 rounding of the difference), and the oracle's
    update where the gradient is well above rounding noise.  At step 1 Adam moves
    every weight by ~lr * sign(g) whatever |g| is, so on near-zero gradients the
    sign is rounding noise; those elements are left to the moment checks."""
    w0, w1, dm, dv = (np.asarray(a, np.float64) for a in (w0, w1, dm, dv))
    u = w1 - w0
    want = -lr * (dm / (1 - beta1 ** step)) / (np.sqrt(dv / (1 - beta2 ** step)) + eps)
    # w1 and w0 are f32: their difference carries one ulp of |w| each
    slack = 2 * np.spacing(np.maximum(np.abs(w0), np.abs(w1)).astype(np.float32)).astype(np.float64)
    err = np.max(np.abs(u - want) - slack)
    print(f"  {name}: update vs closed form on the device's moments: max excess {err:.2e} (lr {lr:g})", flush=True)
    assert err <= 1e-5 * lr, f"{name}: update deviates from the Adam closed form by {err:.3e}"
    ref_dm = np.asarray(ref_dm, np.float64)
    sel = np.abs(ref_dm) >= 1e-2 * np.max(np.abs(ref_dm))
    return check(f"{name} (|g| >= 1e-2 max|g|)", u[sel], np.asarray(ref_update, np.float64)[sel], FP16_TOL)


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def he_normal(g: np.random.Generator, fan_in: int, fan_out: int) -> np.ndarray:
    return (g.standard_normal((fan_in, fan_out)) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
