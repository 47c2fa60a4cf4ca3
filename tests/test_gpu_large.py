"""Parity at shapes that select the 256x256 fp16 tiles (>= 192 output tiles) and the
128x128 fp32 tiles, one GEMM kind at a time so the oracle finishes in seconds."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import FP16_TOL, FP32_TOL, f16, he_normal, normwise, rng

pytestmark = pytest.mark.gpu

BIG = 3584   # 14 x 256: 196 output tiles of 256 x 256


def pair(ctx, K, N, M, half, seed, act=abi.ACT_SILU):
    g = rng(seed)
    w = he_normal(g, K, N)
    ob = O.OracleBlock(K, N, M, w, half=half, act=act, master_w=w if half else None)
    db = DeviceBlock(ctx, K, N, M, w, half=half, act=act, master_w=w if half else None)
    return ob, db


def up(x, half):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda().to(torch.float16 if half else torch.float32)


@pytest.mark.parametrize("half,M,K,N", [(True, BIG, 256, BIG), (False, 2048, 256, 2048)])
def test_forward_large_tiles(ctx, half, M, K, N):
    ob, db = pair(ctx, K, N, M, half, 1)
    x = rng(2).standard_normal((M, K)).astype(np.float32)
    x = f16(x) if half else x
    ob.forward(x, M)
    db.forward(up(x, half), M)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    for n in ("preact", "out"):
        e = normwise(db.get(n), getattr(ob, n))
        assert e <= tol, f"{n}: {e:.3e}"


@pytest.mark.parametrize("half,M,K,N", [(True, BIG, BIG, 256), (False, 2048, 2048, 256)])
def test_input_grad_large_tiles(ctx, half, M, K, N):
    ob, db = pair(ctx, K, N, M, half, 3)
    x = rng(4).standard_normal((M, K)).astype(np.float32)
    x = f16(x) if half else x
    ob.forward(x, M)
    db.forward(up(x, half), M)
    s = (rng(5).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    dx = db.input_grad(M)
    torch.cuda.synchronize()
    e = normwise(dx.cpu().numpy(), ob.input_grad(M))
    assert e <= (FP16_TOL if half else FP32_TOL), f"input_grad: {e:.3e}"


@pytest.mark.parametrize("half,M,K,N", [(True, 256, BIG, BIG), (False, 256, 2048, 2048)])
def test_backward_large_tiles(ctx, half, M, K, N):
    ob, db = pair(ctx, K, N, M, half, 6)
    x = rng(7).standard_normal((M, K)).astype(np.float32)
    x = f16(x) if half else x
    ob.forward(x, M)
    db.forward(up(x, half), M)
    s = (rng(8).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    ob.backward(x, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), M, 0.01, 3.4e38, 1)
    db.backward(up(x, half), abi.train_ctx(abi.sgd(0.0), abi.sgd(0.0), M, 0.01), 1)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    for n in ("dv_w", "dv_b"):
        e = normwise(db.get(n), getattr(ob, n))
        assert e <= tol, f"{n}: {e:.3e}"
