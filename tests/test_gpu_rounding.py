"""Rounding points of fp16 blocks on the device, checked bit for bit on the device's own values.

forward.cu:61-72 with T = half: rstd = T(rsqrt(sum z^2 / N + 1e-6)) is stored in
T, and preact = T(T(prenorm * rstd) * norm_w) is computed in half arithmetic,
one rounding per product.  The product of two fp16 values is exact in fp32
(11 + 11 significand bits), so that expression is f16(f16(z * r) * g) with the
products in float32.  The test reads the device's prenorm, norm_rstd, norm_w and
preact and requires that equality element by element, and it checks that the
alternatives a kernel could plausibly compute instead (one rounding of z r g, or
the fp32 rstd in place of its fp16 rounding) differ from the device's preact on
a share of the elements, so the equality is not met by accident.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import f16, he_normal, rng

pytestmark = pytest.mark.gpu


def h(x) -> np.ndarray:
    """Round float32 to fp16 (nearest even) and back."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("M,K,N", [
    (192, 256, 384),    # widths a multiple of 4: the row-in-registers norm kernel
    (97, 64, 1531),     # odd width: the aligned-group norm kernel
    (16, 32, 4093),
])
def test_rms_forward_fp16_double_rounding(ctx, M, K, N):
    print(f"[case] fp16 RMSNorm forward M={M} K={K} N={N}", flush=True)
    g = rng(M + N)
    w = he_normal(g, K, N)
    db = DeviceBlock(ctx, K, N, M, w, half=True, norm=abi.NORM_RMS, act=abi.ACT_IDENTITY, master_w=w)
    gw = h(0.5 + g.random((1, N)).astype(np.float32))   # norm weight away from 1, in fp16
    db.norm_w.copy_(torch.from_numpy(gw).cuda().half())
    db.master_norm_w.copy_(torch.from_numpy(gw).cuda())
    x = torch.from_numpy(f16(g.standard_normal((M, K)).astype(np.float32))).cuda().half()
    db.forward(x, M)
    torch.cuda.synchronize()
    z = db.get("prenorm")[:M]
    r = db.get("norm_rstd")[:M].reshape(M, 1)
    pre = db.get("preact")[:M]
    # the stored rstd is the fp16 rounding of rsqrt(mean z^2 + 1e-6) (within one fp16 ulp:
    # the device sums the squares in its own order)
    r64 = 1.0 / np.sqrt(np.mean(z.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    assert np.all(np.abs(r - r64) <= np.spacing(h(r64).astype(np.float16)).astype(np.float64) * 1.01)
    twice = h(h(z * r) * gw)
    bad = int(np.sum(pre.view(np.uint32) != twice.view(np.uint32)))
    print(f"  preact != f16(f16(z r) g): {bad} of {pre.size} elements", flush=True)
    assert bad == 0
    once = h(z.astype(np.float64) * r * gw)
    r32 = h(z * (1.0 / np.sqrt(np.mean(z * z, axis=1, keepdims=True) + np.float32(1e-6))).astype(np.float32)) * gw
    n_once, n_r32 = int(np.sum(once != pre)), int(np.sum(h(r32) != pre))
    print(f"  single rounding differs at {n_once}, fp32 rstd at {n_r32} elements", flush=True)
    assert n_once > pre.size // 100 and n_r32 > pre.size // 100
