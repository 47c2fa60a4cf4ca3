"""The hidden-layer error fused into the 256x256 dX GEMM (fp16).

compute_hidden_layer_error_kernel (backward.cu:59-102) is one kernel in the
reference: the dX sum and its epilogue.  Here too, when the hidden error's
output is whole 256x256 tiles with 4-aligned rows and aligned buffers: the
GEMM's epilogue computes e = mask * act'(s, ...), grad, the element-local norm
gradient into d_prenorm / d_prenorm_h / dNorm and each 256-row tile's column
sums, which the backward that follows takes for db and the norm-parameter
sums.  Ragged outputs and misaligned buffers take the GEMM + error-kernel pair
instead, and a next layer of at most 16 outputs the error kernel that forms the
sum itself; all three kinds are here.  Checked against the oracle (fed the device's
forward caches) at shapes that select the 256x256 kernel: every norm mode
(BatchNorm with its per-column rstd), dropout masks, and the parameters after
backward_hidden (the column sums' only consumer).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from tests.helpers import FP16_TOL, f16, rng
from tests.test_gpu_configs import sync_caches
from tests.test_gpu_parity import check, dev, inputs, make_pair
from tests.test_gpu_unaligned import misalign

pytestmark = pytest.mark.gpu

CASES = [
    # (M, K0, N0, N1, norm, act, dropout p, buffer offset)
    (4096, 64, 3072, 512, abi.NORM_RMS, abi.ACT_MISH, 0.1, 0),     # C4's recipe, whole tiles
    (4096, 64, 3072, 512, abi.NORM_LAYER, abi.ACT_LEAKY, 0.0, 0),
    (4096, 64, 3072, 512, abi.NORM_BATCH, abi.ACT_TANH, 0.0, 0),   # rstd per column, 1/m
    (4096, 64, 3072, 512, abi.NORM_DISABLED, abi.ACT_SILU, 0.2, 0),
    (4001, 64, 3001, 13, abi.NORM_LAYER, abi.ACT_LEAKY, 0.0, 0),   # ragged, K 13: error kernel forms the sum
    (4001, 64, 3001, 777, abi.NORM_RMS, abi.ACT_SIGMOID, 0.0, 0),  # ragged: GEMM + error kernel
    (4096, 64, 3072, 512, abi.NORM_RMS, abi.ACT_MISH, 0.0, 1),     # buffers off 16 bytes: GEMM + error kernel
    (4096, 64, 3072, 512, abi.NORM_LAYER, abi.ACT_RELU, 0.0, 3),
]


@pytest.mark.parametrize("M,K0,N0,N1,norm,act,p,off", CASES)
def test_fused_hidden_error_and_backward(ctx, M, K0, N0, N1, norm, act, p, off):
    print(f"fused hidden error M={M} {N0} <- {N1} norm={norm} act={act} p={p} offset={off}", flush=True)
    o0, d0 = make_pair(ctx, K0, N0, M, seed=N0 + N1 + norm, half=True, norm=norm, act=act, leaky=0.01, p=p)
    o1, d1 = make_pair(ctx, N0, N1, M, seed=N1 + 7, half=True, act=abi.ACT_IDENTITY)
    if off:
        misalign(d0, off)
    x = inputs(101, M, K0, True)
    seed = O.scramble_seed(3, 27)
    o0.forward(x, M, p > 0, seed)
    d0.forward(dev(x, True), M, p > 0, seed)
    o1.forward(o0.out, M)
    d1.forward(d0.out, M)
    torch.cuda.synchronize()
    if p > 0:
        assert np.array_equal(d0.get("mask"), o0.mask), "dropout mask differs"
    # the backward is judged on the device's forward caches: pre-activations
    # within the forward's accumulation noise of 0 flip ReLU' / LeakyReLU'
    sync_caches(o0, d0)
    sync_caches(o1, d1)
    t = (rng(102).random((M, N1)) > 0.5).astype(np.float32)
    o1.output_error(t, abi.LOSS_BCE, abi.ACT_SIGMOID)
    d1.output_error(dev(t, True), abi.LOSS_BCE, abi.ACT_SIGMOID)
    o0.hidden_error(o1, M)
    o0.backward(x, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    d0.backward_hidden(d1, dev(x, True), abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)
    torch.cuda.synchronize()
    for n in ["grad", "d_prenorm"] + (["d_norm_w", "d_norm_b"] if norm else []):
        check(n, d0.get(n), getattr(o0, n), FP16_TOL)
    assert np.array_equal(d0.get("d_prenorm_h"), f16(d0.get("d_prenorm")))
    # db and the norm-parameter sums come from the epilogue's column sums
    names = (["dm_b", "dv_b", "master_b"] if norm != abi.NORM_BATCH else []) + ["dm_w"]
    names += ["dm_norm_w", "master_norm_w"] if norm else []
    names += ["dm_norm_b"] if norm >= abi.NORM_LAYER else []
    for n in names:
        check(n, d0.get(n), getattr(o0, n), FP16_TOL)
