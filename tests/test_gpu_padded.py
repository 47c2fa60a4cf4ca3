"""Parity of the GEMM paths that ragged and small-grid shapes take on the 256x256 fp16
kernel, each at a moderate size the oracle finishes in a second or two:

  * operands the kernel cannot read in place (M, N not whole 256 tiles, K not a
    multiple of 128, rows not 16-byte aligned) are zero-padded into the workspace
    and the epilogue stops at the real M x N, element by element;
  * dW grids smaller than the CU count split the batch over workgroups and the
    optimiser kernel reduces the fp32 partial planes;
  * the hidden error is the dX GEMM into the workspace, then the error kernel.

Gates as everywhere: fp16 2e-2 normwise (elementwise reported) against the oracle; dropout masks bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from tests.helpers import FP16_TOL, rng
from tests.test_gpu_parity import check, dev, inputs, make_pair

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K,N,norm,act,p", [
    (3001, 777, 4001, 0, abi.ACT_SILU, 0.2),      # padded A and B, fused act + dropout epilogue
    (3001, 777, 4001, 2, abi.ACT_LEAKY, 0.0),     # padded, prenorm epilogue then LayerNorm
    (4096, 1000, 3072, 1, abi.ACT_MISH, 0.1),     # only A padded (K % 128), whole output tiles
])
def test_forward_padded(ctx, M, K, N, norm, act, p):
    print(f"forward padded {M}x{K}x{N} norm {norm}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=M + N, half=True, norm=norm, act=act, leaky=0.01, p=p)
    x = inputs(71, M, K, True)
    seed = O.scramble_seed(2, 27)
    ob.forward(x, M, p > 0, seed)
    db.forward(dev(x, True), M, p > 0, seed)
    torch.cuda.synchronize()
    for n in ["preact", "predrop", "out"] + (["prenorm", "centered"] if norm else []):
        check(n, db.get(n)[:M], getattr(ob, n)[:M], FP16_TOL)
    if p > 0:
        assert np.array_equal(db.get("mask")[:M], ob.mask[:M]), "dropout mask differs"


@pytest.mark.parametrize("M,K0,N0,N1,norm", [(4001, 64, 3001, 13, 2), (4001, 64, 3001, 777, 0)])
def test_hidden_error_padded(ctx, M, K0, N0, N1, norm):
    """dX GEMM with K = N1 (13 pads to 128) and a ragged output, then the error kernel
    on unaligned rows (one column per lane), column sums left for the backward."""
    print(f"hidden error padded {M}: {N0} <- {N1} norm {norm}", flush=True)
    o0, d0 = make_pair(ctx, K0, N0, M, seed=81, half=True, norm=norm, act=abi.ACT_LEAKY, leaky=0.01)
    o1, d1 = make_pair(ctx, N0, N1, M, seed=82, half=True, act=abi.ACT_IDENTITY)
    x = inputs(83, M, K0, True)
    o0.forward(x, M)
    d0.forward(dev(x, True), M)
    o1.forward(o0.out, M)
    d1.forward(d0.out, M)
    t = (rng(84).random((M, N1)) > 0.5).astype(np.float32)
    o1.output_error(t, abi.LOSS_BCE, abi.ACT_SIGMOID)
    d1.output_error(dev(t, True), abi.LOSS_BCE, abi.ACT_SIGMOID)
    o0.hidden_error(o1, M)
    o0.backward(x, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    d0.backward_hidden(d1, dev(x, True), abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)
    torch.cuda.synchronize()
    for n in ["grad", "d_prenorm", "dm_b"] + (["d_norm_w", "d_norm_b", "dm_norm_w", "dm_norm_b"] if norm else []):
        check(n, d0.get(n), getattr(o0, n), FP16_TOL)


def test_input_grad_padded(ctx):
    M, K, N = 4001, 3001, 777
    print(f"input grad padded {M}x{K}x{N}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=91, half=True, act=abi.ACT_SILU)
    x = inputs(92, M, K, True)
    ob.forward(x, M)
    db.forward(dev(x, True), M)
    s = (rng(93).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    dx = db.input_grad(M)
    torch.cuda.synchronize()
    check("input_grad", dx.cpu().numpy(), ob.input_grad(M), FP16_TOL)


@pytest.mark.parametrize("M,K,N,norm", [
    (6000, 1000, 1531, 2),   # 24 padded tiles: split-K over the batch, partial planes reduced
    (2048, 2048, 2048, 0),   # 64 whole tiles, operands read in place: split-K only
    (300, 4000, 3001, 1),    # 192 padded tiles, no split: Adam in the element-wise epilogue
])
def test_backward_padded_and_split(ctx, M, K, N, norm):
    print(f"backward {M}: {K}x{N} norm {norm}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=K + N, half=True, norm=norm, act=abi.ACT_SILU)
    x = inputs(101, M, K, True)
    ob.forward(x, M)
    db.forward(dev(x, True), M)
    s = (rng(102).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    ob.backward(x, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    db.backward(dev(x, True), abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)
    torch.cuda.synchronize()
    for n in ("dm_w", "dv_w", "master_w", "dm_b"):
        check(n, db.get(n), getattr(ob, n), FP16_TOL)
    if norm:
        check("dm_norm_w", db.get("dm_norm_w"), ob.dm_norm_w, FP16_TOL)
    assert np.array_equal(db.get("w"), db.get("master_w").astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("M,K,N", [(2048, 1024, 1024), (333, 200, 150)])
def test_gemm_timing_hook(ctx, M, K, N):
    """skl_ctx_time_next_gemm: the next GEMM kernel's dispatch records the two events
    (the 256x256 kernel, then the register-staged one); the call's results are unchanged."""
    print(f"timing hook {M}x{K}x{N}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=5, half=True, act=abi.ACT_SILU)
    x = inputs(6, M, K, True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()   # torch creates its HIP events on first record
    stop.record()
    torch.cuda.synchronize()
    ctx.time_next_gemm(start, stop)
    ob.forward(x, M)
    db.forward(dev(x, True), M)
    stop.synchronize()
    ms = start.elapsed_time(stop)
    assert 0.0 < ms < 1000.0, f"GEMM time {ms} ms"
    torch.cuda.synchronize()
    check("out", db.get("out"), ob.out, FP16_TOL)
