"""Parity at the full sizes of the BASELINE configurations, one training step each,
against the oracle on the same seeded inputs (the oracle finishes each in seconds on
the GPU box's host cores).

  C2  fp32 DenseBlock X[4096 x 1024] -> 1024, ReLU, SGD            (single block)
  C3  fp16 DenseBlock X[8192 x 4096] -> 4096, SiLU, Adam           (single block, headline)
  C4  fp16 MLP 16384 x 3072 -> 2048 -> 2048 -> 2048 -> 2048 -> 10, RMSNorm + Mish +
      dropout 0.1 hidden, CE / Softmax, Adam                       (ffn.rs order, Q1)
  C5  fp16 MLP 12345 x 777 -> 1531 -> 3001 -> 13, LayerNorm + LeakyReLU(0.01) hidden,
      BCE / Sigmoid, Adam                                          (ragged shapes)

Single blocks take one step of forward -> act' of a supplied upstream gradient ->
dW + optimiser -> dX (bench.py's step); the MLPs take FeedForwardNetwork's step.
Gates as everywhere (tests/helpers.py): fp32 1e-4 normwise and 1e-2 elementwise, fp16 2e-2 normwise; dropout
masks bit-exact.

Each stage is checked on identical inputs: after the forward has been compared, the
device's forward caches are copied into the oracle blocks before the backward.  At
these sizes some pre-activations lie within the accumulation-order noise of 0, where
ReLU' / LeakyReLU' jump; one such element differs by the whole upstream value, which
is a property of the discontinuity, not of either implementation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import FP16_TOL, FP32_TOL, check, check_adam_update, check_sum_bound, f16, he_normal, rng
from tests.test_gpu_ffn import build_net

pytestmark = pytest.mark.gpu

CACHES = ("out", "predrop", "preact", "centered", "prenorm", "norm_rstd", "mask")


def sync_caches(ob, db):
    """Give the oracle block the device's forward caches (the backward's inputs)."""
    for n in CACHES:
        setattr(ob, n, np.ascontiguousarray(db.get(n), np.float32).reshape(getattr(ob, n).shape))


def single_block_step(ctx, M, K, N, half, act, opt_o, opt_d, lr):
    g = rng(1000 + M)
    w = he_normal(g, K, N)
    b = (g.standard_normal((1, N)) * 0.01).astype(np.float32)
    if half:
        b = f16(b)
    x = g.standard_normal((M, K)).astype(np.float32)
    x = f16(x) if half else x
    s = (g.standard_normal((M, N)) * 512).astype(np.float32)
    kw = dict(half=half, act=act, b=b, master_w=w if half else None)
    ob = O.OracleBlock(K, N, M, w, **kw)
    db = DeviceBlock(ctx, K, N, M, w, **kw)
    print(f"forward {M}x{K}x{N}", flush=True)
    xd = torch.from_numpy(x).cuda()
    xd = xd.half() if half else xd
    ob.forward(x, M)
    db.forward(xd, M)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    for n in ("preact", "out"):
        check(n, db.get(n), getattr(ob, n), tol)
    sync_caches(ob, db)
    print("backward", flush=True)
    # a single block: dX with the forward's W, then the optimiser step
    ob.error_from_sum(s, M)
    dx_ref = ob.input_grad(M)
    ob.backward(x, opt_o, opt_o, M, lr, 3.4e38, 1)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    dx = db.input_grad(M)
    db.backward(xd, abi.train_ctx(opt_d, opt_d, M, lr), 1)
    torch.cuda.synchronize()
    ob.x_, ob.s_ = x, s
    return ob, db, dx.cpu().numpy(), dx_ref, w


def test_c2_fp32_full_size(ctx):
    tol = FP32_TOL
    M, K, N = 4096, 1024, 1024
    ob, db, dx, dx_ref, w0 = single_block_step(ctx, M, K, N, False, abi.ACT_RELU, O.Optimiser.sgd(0.0),
                                               abi.sgd(0.0), 1e-2)
    for n in ("grad", "d_prenorm", "dv_w", "dv_b", "w", "b"):
        check(n, db.get(n), getattr(ob, n), tol)
    check("dX", dx, dx_ref, tol)
    # element by element, against the summation-error scale of each GEMM output (the sum
    # over k of |a_k b_k|): the north star's 1e-4 relative, with a denominator that the
    # order of the additions cannot exceed
    absx, absw = np.abs(ob.x_).astype(np.float64), np.abs(w0).astype(np.float64)
    check_sum_bound("preact", db.get("preact"), ob.preact, absx @ absw + np.abs(ob.b))
    dp = np.abs(ob.d_prenorm).astype(np.float64)
    check_sum_bound("dX", dx, dx_ref, dp @ absw.T)
    # SGD with momentum 0: dv_w = (x^T . d_prenorm) / 512 / M
    check_sum_bound("dv_w", db.get("dv_w"), ob.dv_w, (absx.T @ dp) / 512.0 / M)


def test_c3_fp16_full_size(ctx):
    tol = FP16_TOL
    ob, db, dx, dx_ref, w0 = single_block_step(ctx, 8192, 4096, 4096, True, abi.ACT_SILU, O.Optimiser.adam(),
                                               abi.adam(), 1e-3)
    for n in ("grad", "d_prenorm", "dm_w", "dv_w", "master_w", "dm_b", "master_b"):
        check(n, db.get(n), getattr(ob, n), tol)
    # master_w moves by ~1e-3 against |w| ~ 0.1: its normwise check cannot see the update
    check_adam_update("master_w update", w0, db.get("master_w"), db.get("dm_w"), db.get("dv_w"), 1e-3, 1,
                      ob.master_w - w0, ob.dm_w)
    check("dX", dx, dx_ref, tol)
    # the fp16 working copy is the RNE of the fp32 master after the update
    assert np.array_equal(db.get("w"), f16(db.get("master_w")))


def mlp_step(ctx, dims, M, hidden_kw, loss, loss_act, x, t, use_dropout, seeds):
    """FeedForwardNetwork::forward, compare, then FeedForwardNetwork::backward (ffn.rs:113-166:
    the layer above is updated before the layer below propagates through it)."""
    obs, dbs = build_net(ctx, dims, M, True, hidden_kw, seed=len(dims) * 100 + M)
    w0 = [(ob.master_w.copy(), ob.master_norm_w.copy()) for ob in obs]   # before the step
    L = len(dims) - 1
    print(f"forward MLP {dims} x {M}", flush=True)
    cur_o, cur_d, outs = x, torch.from_numpy(x).cuda().half(), []
    for ob, db, sd in zip(obs, dbs, seeds):
        cur_o = ob.forward(cur_o, M, use_dropout, sd).copy()
        cur_d = db.forward(cur_d, M, use_dropout, sd)
        outs.append(cur_o)
    torch.cuda.synchronize()
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        if use_dropout and i < L - 1:
            assert np.array_equal(db.get("mask"), ob.mask), f"layer {i} dropout mask"
        check(f"layer {i} out", db.get("out"), ob.out, FP16_TOL)
        sync_caches(ob, db)
    outs = [ob.out.copy() for ob in obs]   # layer inputs of the backward: the synced outputs
    print("backward", flush=True)
    opt = O.Optimiser.adam()
    obs[L - 1].output_error(t, loss, loss_act)
    obs[L - 1].backward(outs[L - 2] if L > 1 else x, opt, opt, M, 1e-3, 3.4e38, 1)
    for i in range(L - 2, -1, -1):
        obs[i].hidden_error(obs[i + 1], M)
        obs[i].backward(outs[i - 1] if i > 0 else x, opt, opt, M, 1e-3, 3.4e38, 1)
    xd = torch.from_numpy(x).cuda().half()
    tc = abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3)
    dbs[L - 1].output_error(torch.from_numpy(t).cuda().half(), loss, loss_act)
    dbs[L - 1].backward(dbs[L - 2].out if L > 1 else xd, tc, 1)
    for i in range(L - 2, -1, -1):
        dbs[i].backward_hidden(dbs[i + 1], dbs[i - 1].out if i > 0 else xd, tc, 1)
    torch.cuda.synchronize()
    return obs, dbs, w0


def check_layer_adam(i, ob, db, w0, norm):
    """Every layer's optimiser state after the step: both moments and the master against
    the oracle, and the master's update against Adam's closed form on the device's own
    moments (master_w moves by ~1e-3 against |w| ~ 0.03-0.1, so its normwise check alone
    could not see a wrong or sign-flipped update); the same for the norm weight."""
    for n in ("dm_w", "dv_w", "master_w", "dm_b", "dv_b", "master_b"):
        check(f"layer {i} {n}", db.get(n), getattr(ob, n), FP16_TOL)
    check_adam_update(f"layer {i} master_w update", w0[0], db.get("master_w"), db.get("dm_w"), db.get("dv_w"), 1e-3,
                      1, ob.master_w - w0[0], ob.dm_w)
    if norm:
        for n in ("dm_norm_w", "dv_norm_w", "master_norm_w"):
            check(f"layer {i} {n}", db.get(n), getattr(ob, n), FP16_TOL)
        check_adam_update(f"layer {i} master_norm_w update", w0[1], db.get("master_norm_w"), db.get("dm_norm_w"),
                          db.get("dv_norm_w"), 1e-3, 1, ob.master_norm_w - w0[1], ob.dm_norm_w)
    assert np.array_equal(db.get("w"), f16(db.get("master_w"))), f"layer {i}: W is not the RNE of its master"


def test_c4_fp16_mlp_full_size(ctx):
    dims, M = [3072, 2048, 2048, 2048, 2048, 10], 16384
    g = rng(404)
    x = f16(g.random((M, 3072), dtype=np.float32))
    t = np.zeros((M, 10), np.float32)
    t[np.arange(M), g.integers(0, 10, M)] = 1
    # weight ids of a fp16 training network built in order: 27 tensors per block (Q8)
    seeds = [O.scramble_seed(1, 27 * i) for i in range(len(dims) - 1)]
    obs, dbs, w0 = mlp_step(ctx, dims, M, dict(norm=abi.NORM_RMS, act=abi.ACT_MISH, mask_coeff=0.1),
                            abi.LOSS_CE, abi.ACT_SOFTMAX, x, t, True, seeds)
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        check(f"layer {i} d_prenorm", db.get("d_prenorm"), ob.d_prenorm, FP16_TOL)
        check_layer_adam(i, ob, db, w0[i], i < len(obs) - 1)


def test_c5_fp16_mlp_ragged_full_size(ctx):
    dims, M = [777, 1531, 3001, 13], 12345
    g = rng(505)
    x = f16(g.standard_normal((M, 777)).astype(np.float32) * np.float32(np.sqrt(2.0)))   # variance 2
    t = (g.random((M, 13)) > 0.5).astype(np.float32)
    obs, dbs, w0 = mlp_step(ctx, dims, M, dict(norm=abi.NORM_LAYER, act=abi.ACT_LEAKY, leaky=0.01),
                            abi.LOSS_BCE, abi.ACT_SIGMOID, x, t, False, [0, 0, 0])
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        check(f"layer {i} d_prenorm", db.get("d_prenorm"), ob.d_prenorm, FP16_TOL)
        check_layer_adam(i, ob, db, w0[i], i < len(obs) - 1)
        if i < len(obs) - 1:
            check(f"layer {i} dm_norm_b", db.get("dm_norm_b"), ob.dm_norm_b, FP16_TOL)
