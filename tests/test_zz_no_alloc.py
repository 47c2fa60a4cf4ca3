"""skl_dense_error_from_sum_noalloc: the allocation-free variant of
skl_dense_error_from_sum (no counterpart in the reference).

It must give the same outputs as skl_dense_error_from_sum, bit for bit (same
kernel; only the column partial sums move to the library's per-GPU scratch),
on two calls in a row, the second with a smaller input, made first on a context
of their own that has allocated nothing, with the GPU's free memory unchanged
across each call.  The backward after it recomputes the column sums (the
scratch is shared by every call on the GPU) where the backward after the regular
call takes them from that call: W, its master and moments come out bit for bit
the same (the dW does not use them), the bias and norm parameters within fp32
summation-order noise (1e-6 relative; the two sums add the same terms in
different orders).  A shape whose partial sums exceed the 16 MiB scratch is
rejected with SKL_ERR_ALLOCATION_LIMIT before anything is written.  The call
is also captured into a HIP graph on a caller-owned stream and replayed three
times, each replay checked against the eager call on fresh inputs.
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


def pair(ctx, K, N, M, half, norm, act, seed, ctx_b=None):
    w = he_normal(rng(seed), K, N)
    kw = dict(half=half, norm=norm, act=act, leaky=0.01, master_w=w if half else None)
    a = DeviceBlock(ctx, K, N, M, w, **kw)
    b = DeviceBlock(ctx_b or ctx, K, N, M, w, **kw)
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


def close(a, b, names, rtol=1e-6):
    torch.cuda.synchronize()
    for n in names:
        ta, tb = getattr(a, n), getattr(b, n)
        if ta is None:
            continue
        ta, tb = ta.double(), tb.double()
        err = float((ta - tb).abs().max() / tb.abs().max().clamp_min(1e-30))
        assert err <= rtol, f"{n}: {err:.3e} relative after the allocation-free call's backward"


@pytest.mark.parametrize("cases", CASES, ids=["fp16", "fp32"])
def test_noalloc_matches_error_from_sum_twice(ctx, cases):
    stream = torch.cuda.current_stream()
    fresh = abi.Context(0, 16, stream=stream.cuda_stream)   # has grown no buffer yet
    try:
        for i, (M, K, N, half, norm, act) in enumerate(cases):
            print(f"error_from_sum_noalloc call {i}: M={M} K={K} N={N} half={half} norm={norm} act={act}",
                  flush=True)
            ref, got, x = pair(ctx, K, N, M, half, norm, act, seed=10 + i, ctx_b=fresh)
            s = torch.from_numpy((rng(20 + i).standard_normal((M, N)) * 512).astype(np.float32)).cuda()
            opt = abi.adam() if half else abi.sgd(0.9)
            tc = abi.train_ctx(opt, opt, M, 1e-3)
            # the regular call and its backward (column sums taken from the error call)
            ref.error_from_sum(s, M)
            ref.backward(x, tc, 1)
            torch.cuda.synchronize()
            free0 = torch.cuda.mem_get_info()[0]
            got.error_from_sum_noalloc(s, M)
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, "the allocation-free call changed the GPU's free memory"
            same(ref, got, OUTS)
            got.backward(x, tc, 1)   # column sums recomputed
            same(ref, got, ("w", "master_w", "dv_w", "dm_w"))
            close(ref, got, ("b", "norm_w", "norm_b", "master_b", "dv_b", "dm_b", "dv_norm_w", "dm_norm_w",
                             "dv_norm_b", "dm_norm_b"))
    finally:
        torch.cuda.synchronize()
        fresh.close()


def test_noalloc_under_graph_capture(ctx):
    """Captured on a caller-owned stream (synchronous context: the call skips its
    synchronisation while the stream captures) and replayed three times, with eager work
    and synchronisations between the replays; every replay equals the eager call."""
    M, K, N = 512, 64, 384
    side = torch.cuda.Stream()
    cap = abi.Context(0, 16, stream=side.cuda_stream)
    try:
        ref, got, x = pair(ctx, K, N, M, True, abi.NORM_LAYER, abi.ACT_SILU, seed=31, ctx_b=cap)
        torch.cuda.synchronize()
        s = torch.zeros((M, N), device="cuda")
        with torch.cuda.stream(side):
            got.error_from_sum_noalloc(s, M)   # outside the capture first
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
            got.error_from_sum_noalloc(s, M)
        torch.cuda.synchronize()
        for rep in range(3):
            s.copy_(torch.from_numpy((rng(40 + rep).standard_normal((M, N)) * 512).astype(np.float32)))
            for n in OUTS:
                getattr(got, n).fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            ref.error_from_sum(s, M)
            same(ref, got, OUTS)
            print(f"  replay {rep}: outputs equal the eager call", flush=True)
    finally:
        torch.cuda.synchronize()
        cap.close()


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
