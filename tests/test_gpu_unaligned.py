"""Parity of the error and norm kernels on rows that do not start on a 4-element boundary.

Output widths with n % 4 != 0 on aligned buffers take the flat error kernel: a
band of 4 / gcd(n, 4) rows is a whole number of aligned 4-element chunks, and
widths under 4 put one chunk across several rows; batches that are not a
multiple of the band end in a partial band done element by element.  Buffers
whose base pointers sit 1..3 elements past a 16-byte boundary (torch views into
a larger allocation) take the 4-column-group path that reads aligned chunks and
splits its stores at chunk boundaries.  The column sums either path leaves feed
the backward's bias and norm-parameter update, checked through the moments.

Gates as everywhere: fp32 1e-4 normwise and 1e-2 elementwise, fp16 2e-2 normwise against the oracle.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from tests.helpers import FP16_TOL, FP32_TOL, f16, rng
from tests.test_gpu_parity import check, dev, inputs, make_pair

pytestmark = pytest.mark.gpu

CACHES = ("out", "predrop", "preact", "centered", "prenorm", "mask", "grad", "d_prenorm", "d_norm_w", "d_norm_b",
          "d_prenorm_h")


def misalign(db, off: int) -> None:
    """Move the block's per-element buffers to views starting `off` elements past an aligned allocation."""
    for name in CACHES:
        t = getattr(db, name)
        if t is None:
            continue
        buf = torch.zeros(t.numel() + 8, device=t.device, dtype=t.dtype)
        view = buf[off:off + t.numel()].view(t.shape)
        view.copy_(t)
        setattr(db, name, view)


def _run(ctx, half, M, K, N, norm, act, off):
    ob, db = make_pair(ctx, K, N, M, seed=N + off, half=half, norm=norm, act=act, leaky=0.01)
    if off:
        misalign(db, off)
    x = inputs(61, M, K, half)
    ob.forward(x, M)
    db.forward(dev(x, half), M)
    s = (rng(62).standard_normal((M, N)) * 512).astype(np.float32)
    s_dev = torch.from_numpy(s).cuda()
    if off:   # the supplied sum misaligned too
        sb = torch.zeros(M * N + 8, device="cuda", dtype=torch.float32)
        s_view = sb[off:off + M * N].view(M, N)
        s_view.copy_(s_dev)
        s_dev = s_view
    print(f"error_from_sum {M}x{N} half={half} norm={norm} offset={off}", flush=True)
    ob.error_from_sum(s, M)
    abi.call("skl_dense_error_from_sum", ctx.h, C.byref(db.desc()), C.c_void_p(s_dev.data_ptr()), M)
    ob.backward(x, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    db.backward(dev(x, half), abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    names = ("grad", "d_prenorm") + (("dm_b",) if norm != 3 else ())
    names += ("d_norm_w", "d_norm_b", "dm_norm_w", "dm_norm_b") if norm else ()
    for n in names:
        check(n, db.get(n), getattr(ob, n), tol)
    if half:
        assert np.array_equal(db.get("d_prenorm_h"), f16(db.get("d_prenorm"))), "d_prenorm_h != f16(d_prenorm)"


@pytest.mark.parametrize("half", [True, False])
@pytest.mark.parametrize("M,K,N,norm,act", [
    (301, 64, 1531, 2, abi.ACT_LEAKY),   # LayerNorm, odd width: row offsets cycle 0, 3, 2, 1
    (300, 64, 1022, 1, abi.ACT_MISH),    # RMSNorm, width 2 mod 4
    (257, 48, 13, 0, abi.ACT_SILU),      # width < 4 columns per group tail
    (64, 32, 1027, 3, abi.ACT_TANH),     # batch norm (per-column statistics)
    (299, 40, 70, 2, abi.ACT_SIGMOID),   # width 2 mod 4 with a last band of one row
])
def test_error_odd_width(ctx, half, M, K, N, norm, act):
    _run(ctx, half, M, K, N, norm, act, 0)


@pytest.mark.parametrize("off", [1, 2, 3])
@pytest.mark.parametrize("half", [True, False])
def test_error_misaligned_buffers(ctx, half, off):
    _run(ctx, half, 130, 64, 1024, 2, abi.ACT_SILU, off)


@pytest.mark.parametrize("half", [True, False])
@pytest.mark.parametrize("M,N,norm", [(515, 13, 2), (203, 1, 0), (130, 2, 0), (77, 3, 1)])
def test_output_error_odd_width(ctx, half, M, N, norm):
    """Widths under 4 put one 4-element chunk across several rows."""
    K = 40
    ob, db = make_pair(ctx, K, N, M, seed=71 + N, half=half, norm=norm)
    x = inputs(72, M, K, half)
    ob.forward(x, M)
    db.forward(dev(x, half), M)
    t = (rng(73).random((M, N)) > 0.5).astype(np.float32)
    print(f"output_error {M}x{N} half={half}", flush=True)
    ob.output_error(t, abi.LOSS_BCE, abi.ACT_SIGMOID)
    db.output_error(dev(t, half), abi.LOSS_BCE, abi.ACT_SIGMOID)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    for n in ("grad", "d_prenorm") + (("d_norm_w", "d_norm_b") if norm else ()):
        check(n, db.get(n), getattr(ob, n), tol)


FWD_CACHES = ("z", "prenorm", "centered", "preact", "predrop", "out", "mask")


@pytest.mark.parametrize("off", [1, 4])
@pytest.mark.parametrize("norm", [1, 2])
def test_forward_norm_misaligned_buffers(ctx, norm, off):
    """The row-norm forward on fp16 caches starting `off` elements past an aligned
    allocation: 4 elements keeps 8-byte groups aligned (aligned-group kernel), 1 does
    not (element kernel)."""
    M, K, N = 203, 48, 1024
    ob, db = make_pair(ctx, K, N, M, seed=81 + off, half=True, norm=norm, act=abi.ACT_SILU, p=0.1)
    for name in FWD_CACHES:
        t = getattr(db, name, None)
        if t is None:
            continue
        buf = torch.zeros(t.numel() + 8, device=t.device, dtype=t.dtype)
        setattr(db, name, buf[off:off + t.numel()].view(t.shape))
    x = inputs(82, M, K, True)
    seed = O.scramble_seed(5, 9)
    print(f"forward norm={norm} offset={off}", flush=True)
    ob.forward(x, M, True, seed)
    db.forward(dev(x, True), M, True, seed)
    torch.cuda.synchronize()
    for n in ("preact", "predrop", "out", "mask", "centered"):
        check(n, db.get(n), getattr(ob, n), FP16_TOL)
