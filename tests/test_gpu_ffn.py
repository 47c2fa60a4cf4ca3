"""Multi-layer train steps (src/ffn.rs:40-166 order) on the GPU against the oracle.

The orchestration below restates FeedForwardNetwork::forward / backward: every
layer forward; compute_loss on the last layer; backward_output on the last
layer (its weights are updated first); then for each lower layer, the hidden
error computed from the ALREADY UPDATED next layer, followed by its own update.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import FP16_TOL, FP32_TOL, check, f16, he_normal, rng

pytestmark = pytest.mark.gpu


def build_net(ctx, dims, M, half, hidden_kw, seed):
    g = rng(seed)
    obs, dbs = [], []
    for i in range(len(dims) - 1):
        K, N = dims[i], dims[i + 1]
        w = he_normal(g, K, N)
        kw = dict(hidden_kw) if i < len(dims) - 2 else dict(act=abi.ACT_IDENTITY)
        obs.append(O.OracleBlock(K, N, M, w, half=half, master_w=w if half else None, **kw))
        dbs.append(DeviceBlock(ctx, K, N, M, w, half=half, master_w=w if half else None, **kw))
    return obs, dbs


def oracle_step(obs, x, t, M, loss, loss_act, opt, lr, step, use_dropout, seeds):
    cur = x
    outs = []
    for ob, sd in zip(obs, seeds):
        cur = ob.forward(cur, M, use_dropout, sd).copy()
        outs.append(cur)
    last = len(obs) - 1
    obs[last].output_error(t, loss, loss_act)
    head_in = outs[last - 1] if last > 0 else x
    obs[last].backward(head_in, opt, opt, M, lr, 3.4e38, step)
    for i in range(last - 1, -1, -1):
        obs[i].hidden_error(obs[i + 1], M)
        obs[i].backward(outs[i - 1] if i > 0 else x, opt, opt, M, lr, 3.4e38, step)


def device_step(dbs, x, t, M, loss, loss_act, opt, lr, step, use_dropout, seeds):
    cur = x
    for db, sd in zip(dbs, seeds):
        cur = db.forward(cur, M, use_dropout, sd)
    last = len(dbs) - 1
    dbs[last].output_error(t, loss, loss_act)
    tc = abi.train_ctx(opt, opt, M, lr)
    head_in = dbs[last - 1].out if last > 0 else x
    dbs[last].backward(head_in, tc, step)
    for i in range(last - 1, -1, -1):
        dbs[i].backward_hidden(dbs[i + 1], dbs[i - 1].out if i > 0 else x, tc, step)


def compare_nets(obs, dbs, M, tol, half):
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        for n in ("out", "preact", "grad", "d_prenorm", "dv_w", "dm_w", "dv_b"):
            check(f"layer {i} {n}", db.get(n), getattr(ob, n), tol)
        wn = "master_w" if half else "w"
        check(f"layer {i} {wn}", db.get(wn), getattr(ob, wn), tol)


def test_c1_mlp_fp32_sgd(ctx):
    """784->128(ReLU)->10(softmax CE), fp32, batch 64, SGD lr 0.01."""
    M = 64
    obs, dbs = build_net(ctx, [784, 128, 10], M, False, dict(act=abi.ACT_RELU), seed=1)
    g = rng(101)
    x = g.random((M, 784), dtype=np.float32)
    lab = g.integers(0, 10, M)
    t = np.zeros((M, 10), np.float32)
    t[np.arange(M), lab] = 1
    seeds = [O.scramble_seed(1, 100 + i) for i in range(2)]
    oracle_step(obs, x, t, M, abi.LOSS_CE, abi.ACT_SOFTMAX, O.Optimiser.sgd(0.0), 0.01, 1, False, seeds)
    device_step(dbs, torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda(), M, abi.LOSS_CE, abi.ACT_SOFTMAX,
                abi.sgd(0.0), 0.01, 1, False, seeds)
    torch.cuda.synchronize()
    compare_nets(obs, dbs, M, FP32_TOL, False)


def test_lib_example_nesterov_dropout(ctx):
    """The reference's own test network (src/lib.rs:64-137): 32-16-8-4 fp32, LeakyReLU(0.01)
    with dropout 0.1 on the hidden layers, CE/Softmax, SGD v=0.9 Nesterov, lr 0.01, on
    seeded (non-zero) inputs so values are checked, not only the absence of errors."""
    M = 64
    obs, dbs = build_net(ctx, [32, 16, 8, 4], M, False, dict(act=abi.ACT_LEAKY, leaky=0.01, mask_coeff=0.1), 2)
    g = rng(102)
    x = g.standard_normal((M, 32)).astype(np.float32)
    t = np.zeros((M, 4), np.float32)
    t[np.arange(M), g.integers(0, 4, M)] = 1
    seeds = [O.scramble_seed(1, 7 + 23 * i) for i in range(3)]
    oracle_step(obs, x, t, M, abi.LOSS_CE, abi.ACT_SOFTMAX, O.Optimiser.sgd(0.9, True), 0.01, 1, True, seeds)
    device_step(dbs, torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda(), M, abi.LOSS_CE, abi.ACT_SOFTMAX,
                abi.sgd(0.9, True), 0.01, 1, True, seeds)
    torch.cuda.synchronize()
    for ob, db in zip(obs[:-1], dbs[:-1]):
        assert np.array_equal(db.get("mask"), ob.mask)
    compare_nets(obs, dbs, M, FP32_TOL, False)


def test_c4_like_rms_mish_dropout_fp16_small(ctx):
    """Scaled-down BASELINE config 4: RMSNorm + Mish + dropout 0.1 hidden layers, CE, Adam, fp16."""
    M = 256
    obs, dbs = build_net(ctx, [96, 64, 64, 10], M, True,
                         dict(norm=abi.NORM_RMS, act=abi.ACT_MISH, mask_coeff=0.1), seed=3)
    g = rng(103)
    x = f16(g.random((M, 96), dtype=np.float32))
    t = np.zeros((M, 10), np.float32)
    t[np.arange(M), g.integers(0, 10, M)] = 1
    seeds = [O.scramble_seed(1, 30 + 27 * i) for i in range(3)]
    oracle_step(obs, x, t, M, abi.LOSS_CE, abi.ACT_SOFTMAX, O.Optimiser.adam(), 1e-3, 1, True, seeds)
    device_step(dbs, torch.from_numpy(x).cuda().half(), torch.from_numpy(t).cuda().half(), M, abi.LOSS_CE,
                abi.ACT_SOFTMAX, abi.adam(), 1e-3, 1, True, seeds)
    torch.cuda.synchronize()
    for ob, db in zip(obs[:-1], dbs[:-1]):
        assert np.array_equal(db.get("mask"), ob.mask)
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        for n in ("out", "d_prenorm", "dm_w", "dv_w"):
            check(f"layer {i} {n}", db.get(n), getattr(ob, n), FP16_TOL)


def test_c5_like_ragged_ln_leaky_bce_fp16_small(ctx):
    """Scaled-down BASELINE config 5: 77->153->301->13, LayerNorm + LeakyReLU(0.01), sigmoid BCE, Adam, fp16."""
    M = 123
    obs, dbs = build_net(ctx, [77, 153, 301, 13], M, True,
                         dict(norm=abi.NORM_LAYER, act=abi.ACT_LEAKY, leaky=0.01), seed=4)
    g = rng(104)
    x = f16(g.standard_normal((M, 77)).astype(np.float32) * np.sqrt(2.0))
    t = (g.random((M, 13)) > 0.5).astype(np.float32)
    seeds = [0, 0, 0]
    oracle_step(obs, x, t, M, abi.LOSS_BCE, abi.ACT_SIGMOID, O.Optimiser.adam(), 1e-3, 1, False, seeds)
    device_step(dbs, torch.from_numpy(x).cuda().half(), torch.from_numpy(t).cuda().half(), M, abi.LOSS_BCE,
                abi.ACT_SIGMOID, abi.adam(), 1e-3, 1, False, seeds)
    torch.cuda.synchronize()
    for i, (ob, db) in enumerate(zip(obs, dbs)):
        for n in ("out", "d_prenorm", "dm_w", "dv_w", "dm_norm_w"):
            check(f"layer {i} {n}", db.get(n), getattr(ob, n), FP16_TOL)
