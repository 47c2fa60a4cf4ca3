"""skl_dense_error_from_sum_noalloc: the allocation-free variant of
skl_dense_error_from_sum (no counterpart in the reference).

It must give the same outputs as skl_dense_error_from_sum, bit for bit (same
kernel; only the column partial sums move to the library's per-GPU scratch),
on two calls in a row, the second with a smaller input; a following
skl_dense_backward must give the same results as after the regular call (it
recomputes the column sums); a shape whose partial sums exceed the 16 MiB
scratch is rejected with SKL_ERR_ALLOCATION_LIMIT before anything is written.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.helpers import he_normal, rng

pytestmark = pytest.mark.gpu

OUTS = ("grad", "d_prenorm", "d_norm_w", "d_norm_b", "d_prenorm_h")


def pair(ctx, K, N, M, half, norm, act, seed):
    w = he_normal(rng(seed), K, N)
    kw = dict(half=half, norm=norm, act=act, leaky=0.01, master_w=w if half else None)
    a = DeviceBlock(ctx, K, N, M, w, **kw)
    b = DeviceBlock(ctx, K, N, M, w, **kw)
    x = torch.from_numpy(rng(seed + 1).standard_normal((M, K)).astype(np.float32)).cuda()
    x = x.half() if half else x
    a.forward(x, M)
    b.forward(x, M)
    return a, b, x


def same(a, b, names):
    torch.cuda.synchronize()
    for n in names:
        ta, tb = getattr(a, n), getattr(b, n)
        if ta is None:
            continue
        assert torch.equal(ta, tb), f"{n} differs between skl_dense_error_from_sum and its allocation-free variant"


# (M, K, N, half, norm, act): the second case of each pair is smaller than the first
CASES = [
    [(2048, 96, 1536, True, abi.NORM_LAYER, abi.ACT_SILU), (300, 96, 1001, True, abi.NORM_RMS, abi.ACT_MISH)],
    [(1024, 64, 777, False, abi.NORM_DISABLED, abi.ACT_RELU), (64, 64, 13, False, abi.NORM_BATCH, abi.ACT_TANH)],
]


@pytest.mark.parametrize("cases", CASES, ids=["fp16", "fp32"])
def test_noalloc_matches_error_from_sum_twice(ctx, cases):
    for i, (M, K, N, half, norm, act) in enumerate(cases):
        print(f"error_from_sum_noalloc call {i}: M={M} K={K} N={N} half={half} norm={norm} act={act}", flush=True)
        ref, got, x = pair(ctx, K, N, M, half, norm, act, seed=10 + i)
        s = torch.from_numpy((rng(20 + i).standard_normal((M, N)) * 512).astype(np.float32)).cuda()
        ref.error_from_sum(s, M)
        got.error_from_sum_noalloc(s, M)
        same(ref, got, OUTS)
        # the backward after either call: column sums from the error call vs recomputed
        opt = abi.adam() if half else abi.sgd(0.9)
        tc = abi.train_ctx(opt, opt, M, 1e-3)
        ref.backward(x, tc, 1)
        got.backward(x, tc, 1)
        same(ref, got, ("w", "b", "norm_w", "norm_b", "master_w", "master_b", "dv_w", "dm_w", "dv_b", "dm_b",
                        "dv_norm_w", "dm_norm_w", "dv_norm_b", "dm_norm_b"))


def test_noalloc_rejects_partials_beyond_the_scratch(ctx):
    """outputs = 1.5 M with 16 rows: one split of 3 x 1.5 M fp32 partial sums is 18 MB > 16 MiB."""
    M, K, N = 16, 1, 1_500_000
    blk = DeviceBlock(ctx, K, N, M, np.full((K, N), 0.5, np.float32), act=abi.ACT_RELU)
    s = torch.ones((M, N), device="cuda")
    for n in ("grad", "d_prenorm"):
        getattr(blk, n).fill_(3.0)
    torch.cuda.synchronize()
    rc = abi.status("skl_dense_error_from_sum_noalloc", ctx.h, C.byref(blk.desc()), C.c_void_p(s.data_ptr()), M)
    torch.cuda.synchronize()
    assert rc == -3   # SKL_ERR_ALLOCATION_LIMIT
    assert torch.all(blk.grad == 3.0) and torch.all(blk.d_prenorm == 3.0)
    # the allocating entry point takes the same shape
    blk.error_from_sum(s, M)
    torch.cuda.synchronize()
    assert torch.all(blk.grad == 0.0)   # preact = predrop = 0: ReLU' = 0
