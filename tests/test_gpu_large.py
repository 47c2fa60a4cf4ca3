"""Parity at shapes that select the 256x256 fp16 tiles (>= 192 output tiles) and the
128x128 fp32 tiles, one GEMM kind at a time so the oracle finishes in seconds."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import FP16_TOL, FP32_TOL, check, f16, he_normal, rng

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
        check(f"{n}", db.get(n), getattr(ob, n), tol)


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
    check(f"input_grad", dx.cpu().numpy(), ob.input_grad(M), (FP16_TOL if half else FP32_TOL))


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
        check(f"{n}", db.get(n), getattr(ob, n), tol)


# The 256x256 tiles also carry the fused epilogues with dropout, with the
# norm prologue of the next kernel, and the hidden-error epilogue (act' x mask
# and the element-local norm gradient).  Output BIG x BIG, reduction 256.
@pytest.mark.parametrize("norm,act,p", [(0, abi.ACT_SILU, 0.25), (1, abi.ACT_MISH, 0.1), (2, abi.ACT_LEAKY, 0.0)])
def test_forward_large_tiles_dropout_norm(ctx, norm, act, p):
    from tests.test_gpu_parity import check, dev, inputs, make_pair
    M, K, N = BIG, 256, BIG
    ob, db = make_pair(ctx, K, N, M, seed=41, half=True, norm=norm, act=act, leaky=0.01, p=p)
    x = inputs(42, M, K, True)
    seed = O.scramble_seed(5, 9)
    ob.forward(x, M, p > 0, seed)
    db.forward(dev(x, True), M, p > 0, seed)
    torch.cuda.synchronize()
    for n in ["preact", "predrop", "out"] + (["prenorm", "centered"] if norm else []):
        check(n, db.get(n)[:M], getattr(ob, n)[:M], FP16_TOL)
    if p > 0:
        assert np.array_equal(db.get("mask")[:M], ob.mask[:M]), "dropout mask differs"


@pytest.mark.parametrize("norm,act,p", [(0, abi.ACT_SILU, 0.2), (1, abi.ACT_MISH, 0.0), (2, abi.ACT_TANH, 0.1)])
def test_hidden_error_large_tiles(ctx, norm, act, p):
    from tests.test_gpu_parity import check, dev, inputs, make_pair
    M, K0, N0, N1 = BIG, 256, BIG, 256
    o0, d0 = make_pair(ctx, K0, N0, M, seed=51, half=True, norm=norm, act=act, leaky=0.01, p=p)
    o1, d1 = make_pair(ctx, N0, N1, M, seed=52, half=True, act=abi.ACT_IDENTITY)
    x = inputs(53, M, K0, True)
    seed = 777
    o0.forward(x, M, p > 0, seed)
    d0.forward(dev(x, True), M, p > 0, seed)
    o1.forward(o0.out, M)
    d1.forward(d0.out, M)
    t = (rng(54).random((M, N1)) > 0.5).astype(np.float32)
    o1.output_error(t, abi.LOSS_BCE, abi.ACT_SIGMOID)
    d1.output_error(dev(t, True), abi.LOSS_BCE, abi.ACT_SIGMOID)
    o0.hidden_error(o1, M)
    d0.hidden_error(d1, M)
    torch.cuda.synchronize()
    for n in ["grad", "d_prenorm"] + (["d_norm_w", "d_norm_b"] if norm else []):
        check(n, d0.get(n)[:M], getattr(o0, n)[:M], FP16_TOL)
