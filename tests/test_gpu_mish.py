"""Mish and its derivative on fp16 blocks, over every fp16 value in [-30, 30].

fp16 blocks evaluate Mish (util.cu:28-39) and its slope (util.cu:75-87) from
one hardware exp and reciprocal per element, in the form
tanh(softplus(x)) = n / (n + 2) with n = e^x (e^x + 2); fp32 blocks keep the
reference's exp / log / exp form.  The two agree to a few fp32 ulp except as
x -> -inf, where the reference's e^sp - e^-sp cancels.  So each is checked
here against float64 arithmetic: the device's fp16 Mish within 0.6 fp16 ulp
of the exact value and its fp32 slope within 1e-4 of it (relative, floor 1e-3:
the slope crosses zero near x = -1.19, where its two terms cancel to ~1e-8),
and the oracle (the reference's form) within its own, larger error.  The
reference's overflow behaviour is kept: above x = 20 softplus is x itself,
and from the least float whose e^x rounds to +inf (88.7228...) the result is
NaN on both sides.

The block's weights are the identity and its bias zero, so the forward's
pre-activation is X exactly (one non-zero product per fp32 sum) and the
hidden error from a sum of ones is the slope itself.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock

pytestmark = pytest.mark.gpu

EXP_OVERFLOW = np.float32(88.72283935546875)   # least float whose e^x rounds to +inf


def grid(M, K):
    """Every fp16 value in [-30, 30], then large values around the overflow point, tiled to [M x K]."""
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = np.unique(allh[np.isfinite(allh) & (np.abs(allh) <= 30)].astype(np.float32))
    big = np.float16([20.0, 20.02, 44.0, 88.0, 88.6875, 88.75, 89.0, 100.0, 1000.0, 65504.0, -88.75, -1000.0,
                      -65504.0]).astype(np.float32)
    x = np.concatenate([v, big])
    assert x.size <= M * K
    return np.resize(x, M * K).reshape(M, K)


def exact_mish(x):
    xd = x.astype(np.float64)
    t = np.tanh(np.log1p(np.exp(np.minimum(xd, 20.0))))
    t = np.where(xd > 20.0, 1.0, t)
    sig = 1.0 / (1.0 + np.exp(-xd))
    m = np.where(xd > 20.0, xd, xd * t)
    s = np.where(xd > 20.0, 1.0, t + xd * sig * (1.0 - t * t))
    nan = x >= EXP_OVERFLOW
    return np.where(nan, np.nan, m), np.where(nan, np.nan, s)


def test_fp16_mish_and_slope_exact_over_fp16_range(ctx):
    M = K = N = 256
    x = grid(M, K)
    w = np.eye(K, N, dtype=np.float32)
    b = np.zeros((1, N), np.float32)
    kw = dict(half=True, act=abi.ACT_MISH, b=b)
    ob = O.OracleBlock(K, N, M, w, master_w=w, **kw)
    db = DeviceBlock(ctx, K, N, M, w, master_w=w, **kw)
    xd = torch.from_numpy(x).cuda().to(torch.float16)
    print(f"mish grid: {x.size} values, identity {K}x{N}", flush=True)
    ob.forward(x, M)
    db.forward(xd, M)
    torch.cuda.synchronize()
    assert np.array_equal(db.get("preact").astype(np.float32), x), "identity GEMM must reproduce X"
    em, es = exact_mish(x)
    nan = np.isnan(em)
    assert nan.sum() == 5   # 88.75, 89, 100, 1000, 65504

    # forward: fp16 Mish within 0.6 ulp of exact; NaN exactly where the reference's is
    pd = db.get("predrop").astype(np.float32)
    assert np.array_equal(np.isnan(pd), nan) and np.array_equal(np.isnan(ob.predrop), nan)
    fin = ~nan
    ulp = np.spacing(np.abs(em[fin]).astype(np.float16)).astype(np.float64)
    err = np.abs(pd[fin] - em[fin])
    print(f"  mish: max error {np.max(err / ulp):.3f} fp16 ulp", flush=True)
    assert np.all(err <= 0.6 * ulp + 1e-12)
    orc_err = np.abs(ob.predrop[fin] - em[fin]) / ulp
    print(f"  oracle (reference form) mish: max error {orc_err.max():.3f} fp16 ulp", flush=True)

    # backward: the hidden error from a sum of ones is mask * slope = slope
    s = np.ones((M, N), np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    torch.cuda.synchronize()
    dp = db.get("d_prenorm")
    assert np.array_equal(np.isnan(dp), nan) and np.array_equal(np.isnan(ob.d_prenorm), nan)
    den = np.maximum(np.abs(es[fin]), 1e-3)
    e_dev = np.max(np.abs(dp[fin] - es[fin]) / den)
    e_orc = np.max(np.abs(ob.d_prenorm[fin] - es[fin]) / den)
    print(f"  slope: device {e_dev:.2e}, oracle (reference form) {e_orc:.2e} from exact", flush=True)
    assert e_dev <= 1e-4
    assert e_orc <= 1e-3   # the reference form's own cancellation error


def test_fp32_block_keeps_reference_mish(ctx):
    """fp32 blocks evaluate the reference's exp / log / exp form.

    Where that form is well conditioned (x > -4) the device matches the oracle
    within the fp32 gate (1e-4; libm ulps, amplified by the form's partial
    cancellation near x = -4, come to ~1.5e-5); below x = -8 its e^sp - e^-sp cancellation shows as an
    error against exact arithmetic of more than 1e-3 (relative) on the device as
    on the oracle, which the fp16 blocks' form (a few 1e-7) would not have.
    """
    M = K = N = 256
    x = grid(M, K)
    w = np.eye(K, N, dtype=np.float32)
    b = np.zeros((1, N), np.float32)
    ob = O.OracleBlock(K, N, M, w, act=abi.ACT_MISH, b=b)
    db = DeviceBlock(ctx, K, N, M, w, act=abi.ACT_MISH, b=b)
    ob.forward(x, M)
    db.forward(torch.from_numpy(x).cuda(), M)
    s = np.ones((M, N), np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    torch.cuda.synchronize()
    em, es = exact_mish(x)
    for name, d, o, e in (("mish", db.get("predrop"), ob.predrop, em), ("slope", db.get("d_prenorm"), ob.d_prenorm, es)):
        nan = np.isnan(o)
        assert np.array_equal(np.isnan(d), nan), name
        well = ~nan & (x > -4)
        rel = np.max(np.abs(d[well] - o[well]) / np.maximum(np.abs(o[well]), 1e-2))
        deep = (x > -16) & (x < -8)
        err_d = np.max(np.abs(d[deep] - e[deep]) / np.abs(e[deep]))
        err_o = np.max(np.abs(o[deep] - e[deep]) / np.abs(e[deep]))
        print(f"  fp32 {name}: vs oracle (x > -4) {rel:.2e}; error vs exact for -16 < x < -8: device {err_d:.2e}, "
              f"oracle {err_o:.2e}", flush=True)
        assert rel <= 1e-4, name
        assert err_d > 1e-3 and err_o > 1e-3, name
