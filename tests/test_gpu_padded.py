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
from tests.helpers import FP16_TOL, f16, he_normal, rng
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


@pytest.mark.parametrize("norm,act,p", [(0, abi.ACT_SILU, 0.2), (1, abi.ACT_MISH, 0.1), (2, abi.ACT_LEAKY, 0.1),
                                        (3, abi.ACT_SIGMOID, 0.0)])
def test_forward_row_band(ctx, norm, act, p):
    """A ragged forward whose 256x256 grid would leave most of a third round empty
    (12345 x 3001 padded to 12544 x 3072: 588 tiles) runs output rows 0-10751 on
    256x256 tiles and the rest on 128x128 tiles in a second launch.  Together they
    match the oracle; without a norm the GEMM epilogue applies the activation and
    dropout, whose masks stay bit-exact across the band boundary (the hash takes the
    absolute row)."""
    M, K, N = 12345, 200, 3001
    print(f"forward row band {M}x{K}x{N} norm {norm}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=111 + norm, half=True, norm=norm, act=act, leaky=0.01, p=p)
    x = inputs(112, M, K, True)
    seed = O.scramble_seed(3, 5)
    ob.forward(x, M, True, seed)
    db.forward(dev(x, True), M, True, seed)
    torch.cuda.synchronize()
    for n in ["preact", "predrop", "out"] + (["prenorm", "centered"] if norm else []):
        check(n, db.get(n)[:M], getattr(ob, n)[:M], FP16_TOL)
    assert np.array_equal(db.get("mask")[:M], ob.mask[:M]), "dropout mask differs"


def test_input_grad_row_band(ctx):
    """dX of 12345 rows x 3001 inputs (588 padded 256x256 tiles): the banded pair of
    launches, on padded copies of d_prenorm_h (kept in the context) and W."""
    M, K, N = 12345, 3001, 256
    print(f"input grad row band {M}x{K}x{N}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=121, half=True, act=abi.ACT_SILU)
    x = inputs(122, M, K, True)
    ob.forward(x, M)
    db.forward(dev(x, True), M)
    s = (rng(123).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    dx = db.input_grad(M)
    torch.cuda.synchronize()
    check("input_grad", dx.cpu().numpy(), ob.input_grad(M), FP16_TOL)


@pytest.mark.parametrize("M,K,N,norm", [
    (6000, 1000, 1531, 2),   # 24 padded tiles: split-K over the batch, partial planes reduced
    (2048, 2048, 2048, 0),   # 64 whole tiles, operands read in place: split-K only
    (300, 4000, 3001, 1),    # 192 padded tiles, no split: Adam in the element-wise epilogue
    # split-K grids whose (tile, slice) count is not a multiple of 8 keep the tile order
    # (the others are remapped onto the XCDs): 49 tiles x 5 slices on 256x256 ...
    (5632, 1792, 1792, 1),
    # ... and 36 128x128 tiles x 11 slices
    (5632, 768, 768, 2),
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



BLOCK_FIELDS = ("out", "predrop", "preact", "prenorm", "centered", "norm_rstd", "grad", "d_prenorm", "d_prenorm_h",
                "d_norm_w", "d_norm_b", "w", "master_w", "dm_w", "dv_w", "b", "master_b", "dm_b", "dv_b",
                "norm_w", "master_norm_w", "dm_norm_w", "dv_norm_w", "norm_b", "master_norm_b", "dm_norm_b",
                "dv_norm_b")


def test_kept_padded_d_prenorm_bit_exact(ctx, monkeypatch):
    """An odd-width layer's d_prenorm_h is padded once per step, not twice: the GEMM that
    pads it first (the layer's dW) keeps the copy in the context, and the hidden error of
    the layer below, one call later, reads that copy.  Three identical C5-shaped networks
    take the same three FeedForwardNetwork steps: A through backward_hidden (ffn.rs order)
    and C through separate hidden_error / backward calls, both on the session context;
    B through backward_hidden on a context made with SOKLYN_PAD_KEEP=0, whose GEMMs pad
    into the workspace every time.  Every buffer of every block agrees bit for bit after
    each step.  The batch shrinks and grows back (12345, 10001, 12345): a copy of
    another batch's rows is never read."""
    from soklyn_amd.devblock import DeviceBlock
    monkeypatch.setenv("SOKLYN_PAD_KEEP", "0")
    ctx_ws = abi.Context(0, 16)
    monkeypatch.delenv("SOKLYN_PAD_KEEP")
    ctx_ws.set_stream(torch.cuda.current_stream().cuda_stream)   # the session context's stream
    dims, Mmax = [777, 1531, 3001, 13], 12345
    g = rng(606)
    ws = [he_normal(g, dims[i], dims[i + 1]) for i in range(3)]
    hid = dict(norm=abi.NORM_LAYER, act=abi.ACT_LEAKY, leaky=0.01)

    def net(c):
        return [DeviceBlock(c, dims[i], dims[i + 1], Mmax, ws[i], half=True, master_w=ws[i],
                            **(hid if i < 2 else dict(act=abi.ACT_IDENTITY))) for i in range(3)]

    nets = {"A": net(ctx), "B": net(ctx_ws), "C": net(ctx)}
    x = torch.from_numpy(f16(g.standard_normal((Mmax, 777)).astype(np.float32))).cuda().half()
    t = torch.from_numpy((g.random((Mmax, 13)) > 0.5).astype(np.float32)).cuda().half()
    for step, M in enumerate((12345, 10001, 12345), 1):
        print(f"kept pads step {step}: batch {M}", flush=True)
        tc = abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3)
        for name, n in nets.items():
            cur = x[:M]
            for blk in n:
                cur = blk.forward(cur, M)
            n[2].output_error(t[:M], abi.LOSS_BCE, abi.ACT_SIGMOID)
            n[2].backward(n[1].out, tc, step)
            if name == "C":
                n[1].hidden_error(n[2], M)
                n[1].backward(n[0].out, tc, step)
                n[0].hidden_error(n[1], M)
                n[0].backward(x[:M], tc, step)
            else:
                n[1].backward_hidden(n[2], n[0].out, tc, step)
                n[0].backward_hidden(n[1], x[:M], tc, step)
        torch.cuda.synchronize()
        for other in ("A", "C"):
            for i, (a, b) in enumerate(zip(nets[other], nets["B"])):
                for f in BLOCK_FIELDS:
                    ta, tb = getattr(a, f), getattr(b, f)
                    if ta is None:
                        continue
                    bits = torch.int16 if ta.dtype == torch.float16 else torch.int32
                    assert torch.equal(ta.view(bits), tb.view(bits)), f"step {step} net {other} layer {i} {f} differs"
    del nets
    ctx_ws.close()


def test_kept_pad_input_grad_then_backward_bit_exact(ctx, monkeypatch):
    """A single ragged block's step in bench.py's order: error_from_sum, input_grad (its
    dX GEMM pads d_prenorm_h as A and keeps the copy), backward (the dW GEMM reads that
    copy as B one call later).  Against a context with SOKLYN_PAD_KEEP=0 (every GEMM
    pads into the workspace), dx and every buffer agree bit for bit over two steps."""
    from soklyn_amd.devblock import DeviceBlock
    monkeypatch.setenv("SOKLYN_PAD_KEEP", "0")
    ctx_ws = abi.Context(0, 16)
    monkeypatch.delenv("SOKLYN_PAD_KEEP")
    ctx_ws.set_stream(torch.cuda.current_stream().cuda_stream)
    M, K, N = 12345, 1531, 3001   # dX: 294 tiles on the direct-to-LDS kernel, d_prenorm_h padded as A
    g = rng(707)
    w = he_normal(g, K, N)
    blocks = [DeviceBlock(c, K, N, M, w, half=True, master_w=w, act=abi.ACT_SILU) for c in (ctx, ctx_ws)]
    x = dev(inputs(708, M, K, True), True)
    s = torch.from_numpy((g.standard_normal((M, N)) * 512).astype(np.float32)).cuda()
    for step in (1, 2):
        print(f"kept pad dX -> dW step {step}", flush=True)
        tc = abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3)
        dxs = []
        for b in blocks:
            b.forward(x, M)
            b.error_from_sum(s, M)
            dxs.append(b.input_grad(M))
            b.backward(x, tc, step)
        torch.cuda.synchronize()
        assert torch.equal(dxs[0].view(torch.int32), dxs[1].view(torch.int32)), f"step {step} dx differs"
        for f in BLOCK_FIELDS:
            ta, tb = getattr(blocks[0], f), getattr(blocks[1], f)
            if ta is None:
                continue
            bits = torch.int16 if ta.dtype == torch.float16 else torch.int32
            assert torch.equal(ta.view(bits), tb.view(bits)), f"step {step} {f} differs"
    del blocks
    ctx_ws.close()


def test_kept_pad_stale_after_error_call_on_another_context(ctx):
    """Context A's dW pads an odd-width block's d_prenorm_h and keeps the copy; an error
    call on context B then rewrites that d_prenorm_h.  A's next GEMM on it, one call later
    (the input gradient, which would take A's kept copy), must read the new values: its dx
    equals, bit for bit, the one a context that never kept a copy computes."""
    from soklyn_amd.devblock import DeviceBlock
    M, K, N = 12345, 777, 1531   # C5's first layer: zero-padded operands, the dW keeps its copy
    g = rng(707)
    w = he_normal(g, K, N)
    blk = DeviceBlock(ctx, K, N, M, w, half=True, master_w=w, act=abi.ACT_LEAKY, leaky=0.01)
    stream = torch.cuda.current_stream().cuda_stream
    ctx_b = abi.Context(0, 16, stream=stream)
    ctx_c = abi.Context(0, 16, stream=stream)
    try:
        x = torch.from_numpy(f16(g.standard_normal((M, K)).astype(np.float32))).cuda().half()
        s1, s2 = (torch.from_numpy((g.standard_normal((M, N)) * 512).astype(np.float32)).cuda() for _ in range(2))
        blk.forward(x, M)
        blk.error_from_sum(s1, M)
        blk.backward(x, abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)   # pads d_prenorm_h, keeps it
        blk.ctx = ctx_b
        blk.error_from_sum(s2, M)                                            # rewrites it on context B
        blk.ctx = ctx
        dx_a = blk.input_grad(M).cpu().numpy()
        blk.ctx = ctx_c
        dx_c = blk.input_grad(M).cpu().numpy()
        blk.ctx = ctx
        torch.cuda.synchronize()
        assert np.array_equal(dx_a, dx_c), "context A read its stale padded copy of d_prenorm_h"
        print(f"  dx after the rewrite on another context: bit-exact ({dx_a.size} elements)", flush=True)
    finally:
        torch.cuda.synchronize()
        ctx_b.close()
        ctx_c.close()
